"""The captured decode step (q35m_decode_graph_*): one HIP graph of every
layer's mixer plus the length advance, replayed per token.

- A reduced stack (3 Gated-DeltaNet layers + 1 GQA layer, 8 sequences with
  ragged contexts of 441-700 rows) runs 128 steps twice, once by graph replay
  and once by the same launches issued one by one, with new inputs written
  into the graph's fixed input buffers before every step: every layer's
  output is bit-identical between the two after every step, and within 1e-4
  of the oracle, which decodes each sequence at its own moving position; the
  final recurrent states, conv windows and K/V rows match too, and the host
  lengths advanced by 128.
- Host changes to the lengths between replays (truncate, reset, advance,
  snapshot restore) reach the replayed kernels: the graph keeps decoding at
  the new positions, as the oracle does.
- The full 32-layer 4B-shaped stack at batch 1 replays 4 steps within 1e-4
  of the oracle.
- Refusals: a sequence at max_len, a context grown after capture, null
  activations, a layer without weights.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-4 per tensor (fp32); conv
windows and V rows are copies and must match bit for bit.
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


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


class Stack:
    """A context with seeded weights, states and KV rows, the graph's fixed
    activation buffers, and the oracle's copy of every state."""

    def __init__(self, is_rec, n, lens, cap, salt=0):
        self.is_rec, self.n, self.lens = list(is_rec), n, list(lens)
        L = len(is_rec)
        self.c = q35mix.Context(q35mix.qwen35_config(num_layers=L, is_recurrent=self.is_rec), n_seqs=n,
                                kv_capacity=cap)
        c = self.c
        self.w = {}
        self.dn = {}
        self.kv = {}
        for l in range(L):
            if is_rec[l]:
                self.w[l] = synth.deltanet_weights(NK, NV, 128, salt=salt + 60 + l)
                c.set_deltanet_weights(l, self.w[l])
                for s in range(n):
                    st = synth.deltanet_state(NK, NV, 128, salt=salt + 100 * l + s)
                    c.state_write(l, s, q35mix.STATE_RECURRENT, st["state"])
                    c.state_write(l, s, q35mix.STATE_CONV, st["conv_state"])
                    self.dn[l, s] = (st["conv_state"], st["state"])
            else:
                self.w[l] = synth.attn_weights(HD, salt=salt + 60 + l)
                c.set_attn_weights(l, self.w[l])
                for s in range(n):
                    ck = np.zeros((cap, KV_DIM), np.float32)
                    cv = np.zeros_like(ck)
                    if lens[s]:
                        k, v = synth.kv_prefill(lens[s], KV_DIM, salt=salt + 10 * l + s)
                        ck[:lens[s]], cv[:lens[s]] = k, v
                        c.state_write(l, s, q35mix.STATE_KEYS, k)
                        c.state_write(l, s, q35mix.STATE_VALUES, v)
                    self.kv[l, s] = (ck, cv)
        for s in range(n):
            c.advance(s, lens[s])
        self.io = []
        for l in range(L):
            if is_rec[l]:
                self.io.append((c.array((n, c.conv_dim)), c.array((n, c.value_dim)), c.array((n, NV)),
                                c.array((n, NV)), c.array((n, c.value_dim))))
            else:
                self.io.append((c.array((n, 2 * c.q_dim)), c.array((n, c.kv_dim)), c.array((n, c.kv_dim)),
                                None, c.array((n, c.q_dim))))

    def inputs(self, step):
        """Fresh per-(step, layer) inputs, uploaded into the fixed buffers."""
        xs = {}
        for l, rec in enumerate(self.is_rec):
            if rec:
                x = synth.deltanet_inputs(self.n, NK, NV, 128, salt=1000 + 37 * step + l)
                for buf, key in zip(self.io[l][:4], ("qkv", "z", "b", "a")):
                    buf.upload(x[key])
            else:
                x = synth.attn_inputs(self.n, NH, NKV, HD, salt=5000 + 37 * step + l)
                for buf, key in zip(self.io[l][:3], ("q_gate", "k", "v")):
                    buf.upload(x[key])
            xs[l] = x
        return xs

    def outputs(self):
        return [self.io[l][4].download() for l in range(len(self.is_rec))]

    def oracle_step(self, xs, seqs):
        """The oracle's outputs of one step for `seqs`; advances its lengths."""
        outs = {}
        for l, rec in enumerate(self.is_rec):
            x = xs[l]
            for s in seqs:
                if rec:
                    cs, st = self.dn[l, s]
                    o, cs, st, _ = oracle.deltanet_decode(DIMS, x["qkv"][s], x["z"][s], x["b"][s], x["a"][s],
                                                          self.w[l], cs, st)
                    self.dn[l, s] = (cs, st)
                else:
                    ck, cv = self.kv[l, s]
                    o, _, _ = oracle.attn_decode(DIMS, self.lens[s], x["q_gate"][s], x["k"][s], x["v"][s],
                                                 self.w[l], ck, cv, n_threads=8, inplace=True)
                outs[l, s] = o
        for s in seqs:
            self.lens[s] += 1
        return outs

    def check_states(self, seqs):
        c = self.c
        for l, rec in enumerate(self.is_rec):
            for s in seqs:
                if rec:
                    cs, st = self.dn[l, s]
                    assert rel(c.state_read(l, s, q35mix.STATE_RECURRENT), st) <= TOL, (l, s)
                    np.testing.assert_array_equal(c.state_read(l, s, q35mix.STATE_CONV), cs)
                else:
                    ck, cv = self.kv[l, s]
                    n = self.lens[s]
                    assert c.kv_len(s) == n
                    if n:
                        assert rel(c.state_read(l, s, q35mix.STATE_KEYS, n), ck[:n]) <= TOL, (l, s)
                        np.testing.assert_array_equal(c.state_read(l, s, q35mix.STATE_VALUES, n), cv[:n])

    def close(self):
        self.c.close()


def test_graph_replays_match_eager_and_oracle():
    """128 steps of a 3 + 1 layer stack, 8 ragged sequences: graph replay ==
    launch-by-launch run bit for bit, both within 1e-4 of the oracle."""
    n, steps, cap, max_len = 8, 128, 1024, 900
    is_rec = [1, 1, 1, 0]
    lens = [700 - 37 * s for s in range(n)]
    seqs = list(range(n))
    a = Stack(is_rec, n, lens, cap)
    b = Stack(is_rec, n, lens, cap)
    try:
        ga = q35mix.DecodeGraph(a.c, seqs, a.io, max_len)
        gb = q35mix.DecodeGraph(b.c, seqs, b.io, max_len)
        worst = 0.0
        for step in range(steps):
            if step % 32 == 0:
                say(f"graph vs eager: step {step}")
            xs = a.inputs(step)
            b.inputs(step)
            ga.run(replay=True)
            gb.run(replay=False)
            oa, ob = a.outputs(), b.outputs()
            ref = a.oracle_step(xs, seqs)
            for l in range(len(is_rec)):
                np.testing.assert_array_equal(oa[l], ob[l], err_msg=f"step {step} layer {l}")
                for s in seqs:
                    e = rel(oa[l][s], ref[l, s])
                    worst = max(worst, e)
                    assert e <= TOL, (step, l, s, e)
        say(f"128 replays bit-identical to the launch-by-launch run; worst error vs oracle {worst:.2e}")
        for s in seqs:
            assert a.c.kv_len(s) == lens[s] + steps and b.c.kv_len(s) == lens[s] + steps
        a.check_states(seqs)
        for l in range(3):
            for s in seqs:
                np.testing.assert_array_equal(a.c.state_read(l, s, q35mix.STATE_RECURRENT),
                                              b.c.state_read(l, s, q35mix.STATE_RECURRENT))
        ga.close()
        gb.close()
    finally:
        a.close()
        b.close()


def test_graph_follows_host_length_changes():
    """Between replays the host truncates, resets, advances and restores
    sequences; the replayed kernels decode at the new positions."""
    n, cap = 3, 512
    is_rec = [1, 0]
    st = Stack(is_rec, n, [200, 150, 90], cap, salt=7)
    c = st.c
    seqs = list(range(n))
    try:
        g = q35mix.DecodeGraph(c, seqs, st.io, cap)
        step = 0

        def run_and_check(tag):
            nonlocal step
            xs = st.inputs(step)
            g.run()
            out = st.outputs()
            ref = st.oracle_step(xs, seqs)
            for l in range(2):
                for s in seqs:
                    e = rel(out[l][s], ref[l, s])
                    assert e <= TOL, (tag, step, l, s, e)
            step += 1

        for _ in range(3):
            run_and_check("start")
        snap, info = c.snapshot_save(0)
        snap_dn = st.dn[0, 0]
        snap_len = st.lens[0]
        run_and_check("after snapshot")
        # truncate sequence 1 by 20 rows (the DeltaNet state is not rolled back, as in the reference)
        c.truncate(1, st.lens[1] - 20)
        st.lens[1] -= 20
        # reset sequence 2: zero state and window, length 0
        c.reset(2)
        st.lens[2] = 0
        zs = synth.deltanet_state(NK, NV, 128)
        st.dn[0, 2] = (np.zeros_like(zs["conv_state"]), np.zeros_like(zs["state"]))
        for _ in range(2):
            run_and_check("after truncate / reset")
        # advance sequence 2 over 40 rows the host wrote itself
        k, v = synth.kv_prefill(40, KV_DIM, salt=99)
        ck, cv = st.kv[1, 2]
        rows = c.state_read(1, 2, q35mix.STATE_KEYS, st.lens[2])
        vrows = c.state_read(1, 2, q35mix.STATE_VALUES, st.lens[2])
        allk = np.concatenate([rows, k])
        allv = np.concatenate([vrows, v])
        c.state_write(1, 2, q35mix.STATE_KEYS, allk)
        c.state_write(1, 2, q35mix.STATE_VALUES, allv)
        n2 = st.lens[2]
        c.advance(2, 40)
        ck[:n2 + 40], cv[:n2 + 40] = allk, allv
        st.lens[2] += 40
        run_and_check("after advance")
        # restore sequence 0 to the snapshot
        c.snapshot_restore(0, snap, info)
        st.dn[0, 0] = snap_dn
        st.lens[0] = snap_len
        for _ in range(2):
            run_and_check("after restore")
        st.check_states(seqs)
        g.close()
    finally:
        st.close()


def test_graph_full_stack_batch1():
    """The 32-layer 4B-shaped stack (24 DeltaNet + 8 GQA) at batch 1 from a
    2000-row context: 4 replays within 1e-4 of the oracle."""
    is_rec = [(i + 1) % 4 != 0 for i in range(32)]
    st = Stack(is_rec, 1, [2000], 2048, salt=3)
    try:
        g = q35mix.DecodeGraph(st.c, [0], st.io, 2048)
        for step in range(4):
            say(f"32-layer batch-1 graph: step {step}")
            xs = st.inputs(step)
            g.run()
            out = st.outputs()
            ref = st.oracle_step(xs, [0])
            for l in range(32):
                e = rel(out[l][0], ref[l, 0])
                assert e <= TOL, (step, l, e)
        st.check_states([0])
        g.close()
    finally:
        st.close()


def test_graph_refusals():
    n, cap = 2, 64
    st = Stack([1, 0], n, [60, 10], cap, salt=11)
    c = st.c
    try:
        with pytest.raises(q35mix.Q35Error) as e:
            q35mix.DecodeGraph(c, [0, 0], st.io, cap)
        assert e.value.code == q35mix.ERR_INVALID
        with pytest.raises(q35mix.Q35Error) as e:
            q35mix.DecodeGraph(c, [0, 1], st.io, cap + 1)
        assert e.value.code == q35mix.ERR_CAPACITY
        bad = [st.io[0], (st.io[1][0], None, st.io[1][2], None, st.io[1][4])]
        with pytest.raises(q35mix.Q35Error) as e:
            q35mix.DecodeGraph(c, [0, 1], bad, cap)
        assert e.value.code == q35mix.ERR_INVALID
        g = q35mix.DecodeGraph(c, [0, 1], st.io, 62)
        st.inputs(0)
        g.run()
        g.run()                                   # sequence 0 now holds 62 rows
        assert c.kv_len(0) == 62 and c.kv_len(1) == 12
        assert g.try_run() == q35mix.ERR_CAPACITY
        assert c.kv_len(0) == 62 and c.kv_len(1) == 12    # nothing ran
        c.truncate(0, 50)
        g.run()
        assert c.kv_len(0) == 51
        c.grow(128)
        assert g.try_run() == q35mix.ERR_RANGE
        g.close()
        g = q35mix.DecodeGraph(c, [0, 1], st.io, 128)
        g.run()
        assert c.kv_len(0) == 52
        g.close()
    finally:
        st.close()
    fresh = q35mix.Context(q35mix.qwen35_config(num_layers=2, is_recurrent=[1, 0]), n_seqs=1, kv_capacity=16)
    try:
        io = [(fresh.array((1, fresh.conv_dim)), fresh.array((1, fresh.value_dim)), fresh.array((1, NV)),
               fresh.array((1, NV)), fresh.array((1, fresh.value_dim))),
              (fresh.array((1, 2 * fresh.q_dim)), fresh.array((1, fresh.kv_dim)), fresh.array((1, fresh.kv_dim)),
               None, fresh.array((1, fresh.q_dim)))]
        with pytest.raises(q35mix.Q35Error) as e:
            q35mix.DecodeGraph(fresh, [0], io, 16)
        assert e.value.code == q35mix.ERR_INVALID           # no weights
    finally:
        fresh.close()


def test_misaligned_activations_refused():
    """Activation pointers must be 16-byte aligned (the kernels move 16-byte
    vectors): a pointer 4 bytes past an aligned buffer is refused by the
    mixer entry points and by the decode graph."""
    st = Stack([1, 0], 1, [10], 64, salt=13)
    c = st.c
    try:
        base = c.array((1, c.conv_dim + 4))
        bad = q35mix.DeviceView(base, 1, (1, c.conv_dim))
        d = st.io[0]
        with pytest.raises(q35mix.Q35Error) as e:
            c.deltanet_decode(0, [0], bad, d[1], d[2], d[3], d[4])
        assert e.value.code == q35mix.ERR_INVALID and "aligned" in str(e.value)
        abase = c.array((1, 2 * c.q_dim + 4))
        abad = q35mix.DeviceView(abase, 1, (1, 2 * c.q_dim))
        a = st.io[1]
        with pytest.raises(q35mix.Q35Error) as e:
            c.attn_decode(1, [0], abad, a[1], a[2], a[4])
        assert e.value.code == q35mix.ERR_INVALID
        with pytest.raises(q35mix.Q35Error) as e:
            q35mix.DecodeGraph(c, [0], [(bad,) + tuple(d[1:]), a], 64)
        assert e.value.code == q35mix.ERR_INVALID
        assert c.kv_len(0) == 10
    finally:
        st.close()
