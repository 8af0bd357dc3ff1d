"""q35m_load_mixer_weights: the mixers' F32 tensors read from a GGUF file
(written to the published layout by tests/gguf_writer.py under the
reference's tensor names) give a context that decodes like the oracle given
the same weights, and bit-identically to one whose weights were set
directly; a missing or non-F32 tensor is refused, and so are dims that are
not the context's."""
import ctypes
import sys

import numpy as np
import pytest

import gguf_writer as gw
import oracle
import q35mix
import synth

pytestmark = pytest.mark.gpu

NK, NV, NH, NKV, HD = 16, 32, 16, 4, 256


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def tensors(wd, wa, drop=None, as_f16=None):
    t = [gw.f32("blk.0.ssm_conv1d.weight", np.asarray(wd["conv_w"]).reshape(4, -1)),
         gw.f32("blk.0.ssm_a", wd["ssm_a"]), gw.f32("blk.0.ssm_dt.bias", wd["dt_bias"]),
         gw.f32("blk.0.ssm_norm.weight", wd["ssm_norm"]),
         gw.f32("blk.1.attn_q_norm.weight", wa["q_norm"]), gw.f32("blk.1.attn_k_norm.weight", wa["k_norm"])]
    t = [x for x in t if x[0] != drop]
    if as_f16:
        t = [(n, 1, d, np.frombuffer(r, np.float32).astype(np.float16).tobytes()) if n == as_f16 else (n, g, d, r)
             for n, g, d, r in t]
    return t


def test_loaded_weights_decode_identically(tmp_path):
    say("GGUF mixer weights")
    cfg = q35mix.qwen35_config(num_layers=2, is_recurrent=[1, 0])
    wd, wa = synth.deltanet_weights(NK, NV, 128, salt=41), synth.attn_weights(HD, salt=41)
    p = tmp_path / "w.gguf"
    gw.write(p, [("general.architecture", gw.STRING, "qwen35")], tensors(wd, wa))
    g = q35mix.Gguf(p)
    a, b = q35mix.Context(cfg, 1, 16), q35mix.Context(cfg, 1, 16)
    a.load_mixer_weights(g)
    b.set_deltanet_weights(0, wd)
    b.set_attn_weights(1, wa)
    xd = synth.deltanet_inputs(1, NK, NV, 128, salt=43)
    xa = synth.attn_inputs(1, NH, NKV, HD, salt=44)
    outs = []
    for c in (a, b):
        od, oa = c.array((1, c.value_dim)), c.array((1, c.q_dim))
        c.deltanet_decode(0, [0], c.array((1, c.conv_dim), xd["qkv"]), c.array((1, c.value_dim), xd["z"]),
                          c.array((1, NV), xd["b"]), c.array((1, NV), xd["a"]), od)
        c.attn_decode(1, [0], c.array((1, 2 * c.q_dim), xa["q_gate"]), c.array((1, c.kv_dim), xa["k"]),
                      c.array((1, c.kv_dim), xa["v"]), oa)
        outs.append((od.download(), oa.download()))
    for u, v in zip(*outs):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    # oracle leg: zero state, position 0, the weights the file holds
    d = oracle.dims()
    conv_dim = 2 * NK * 128 + NV * 128
    rd, _, _, _ = oracle.deltanet_decode(d, xd["qkv"][0], xd["z"][0], xd["b"][0], xd["a"][0], wd,
                                         np.zeros((conv_dim, 3), np.float32), np.zeros((NV, 128, 128), np.float32))
    z = np.zeros((1, NKV * HD), np.float32)
    ra, _, _ = oracle.attn_decode(d, 0, xa["q_gate"][0], xa["k"][0], xa["v"][0], wa, z, z)
    for got, ref in zip(outs[0], (rd, ra)):
        e = float(np.max(np.abs(got[0].astype(np.float64) - ref)) / np.max(np.abs(ref)))
        say(f"loaded weights vs oracle: rel err {e:.2e}")
        assert e <= 1e-4
    # dims that are not the context's are refused before any copy
    lib = q35mix.lib()
    rec = bytes([1, 0])
    for args in ((2, rec, conv_dim // 2, NV, 128, HD), (2, rec, conv_dim, NV // 2, 128, HD),
                 (2, rec, conv_dim, NV, 64, HD), (2, rec, conv_dim, NV, 128, 128),
                 (1, rec, conv_dim, NV, 128, HD), (2, bytes([1, 1]), conv_dim, NV, 128, HD)):
        r = lib.q35m_load_mixer_weights(ctypes.c_void_p(a.handle), ctypes.c_void_p(g.handle), *args)
        assert r == q35mix.ERR_INVALID, args
    g.close()
    for name, kw, code in (("m.gguf", {"drop": "blk.0.ssm_a"}, q35mix.ERR_RANGE),
                           ("h.gguf", {"as_f16": "blk.1.attn_k_norm.weight"}, q35mix.ERR_UNSUPPORTED)):
        gw.write(tmp_path / name, [], tensors(wd, wa, **kw))
        g = q35mix.Gguf(tmp_path / name)
        with pytest.raises(q35mix.Q35Error) as e:
            a.load_mixer_weights(g)
        assert e.value.code == code
        g.close()
    a.close()
    b.close()
