"""Committed golden fixtures (tests/golden, written by gen_fixtures.py from the
pinned oracle): the CPU oracle must reproduce them, and so must the HIP path."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
import q35mix

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
NAMES = sorted(k[:-4] for k in MANIFEST if k.endswith(".npz"))
SH = MANIFEST["_shapes"]
DIMS = oracle.dims(n_k_heads=SH["deltanet"]["n_k_heads"], n_v_heads=SH["deltanet"]["n_v_heads"],
                   n_heads=SH["attention"]["n_heads"], n_kv_heads=SH["attention"]["n_kv_heads"])


def load(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz")))


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


@pytest.mark.parametrize("name", NAMES)
def test_manifest_hash(name):
    data = open(os.path.join(GOLDEN, f"{name}.npz"), "rb").read()
    assert hashlib.sha256(data).hexdigest() == MANIFEST[f"{name}.npz"]


def _oracle_run(name, f):
    if name == "deltanet_decode":
        out, cs, st, _ = oracle.deltanet_decode(DIMS, f["qkv"][0], f["z"][0], f["b"][0], f["a"][0],
                                                f, f["conv_state"], f["state"])
        return {"out": out, "conv_state_out": cs, "state_out": st}
    if name.startswith("deltanet_prefill"):
        T = f["qkv"].shape[0]
        out, cs, st, _ = oracle.deltanet_prefill(DIMS, T, f["qkv"], f["z"], f["b"], f["a"], f,
                                                 f["state"], f["conv_state"])
        return {"out": out, "conv_state_out": cs, "state_out": st}
    start = f["cache_k"].shape[0]
    T = f["q_gate"].shape[0]
    ck = np.zeros((start + T, f["cache_k"].shape[1]), np.float32)
    cv = np.zeros_like(ck)
    ck[:start], cv[:start] = f["cache_k"], f["cache_v"]
    if name == "attn_decode":
        out, k2, _ = oracle.attn_decode(DIMS, start, f["q_gate"][0], f["k"][0], f["v"][0], f, ck, cv)
        return {"out": out, "k_row": k2[start]}
    out, k2, _ = oracle.attn_prefill(DIMS, start, T, f["q_gate"], f["k"], f["v"], f, ck, cv)
    return {"out": out, "k_rows": k2[start:]}


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    f = load(name)
    for key, val in _oracle_run(name, f).items():
        np.testing.assert_allclose(val.reshape(f[key].shape), f[key], rtol=2e-6, atol=1e-7,
                                   err_msg=f"{name}:{key}")


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_reproduces_fixture(name):
    """The HIP mixers against the fixtures: max|d|/max|ref| <= 1e-4 (fp32 gate);
    conv windows bit-exact."""
    f = load(name)
    cfg = q35mix.qwen35_config(num_layers=2, num_heads=SH["attention"]["n_heads"],
                               num_kv_heads=SH["attention"]["n_kv_heads"],
                               n_k_heads=SH["deltanet"]["n_k_heads"],
                               n_v_heads=SH["deltanet"]["n_v_heads"], is_recurrent=[1, 0])
    with q35mix.Context(cfg, n_seqs=1, kv_capacity=16) as c:
        if name.startswith("deltanet"):
            c.set_deltanet_weights(0, f)
            c.state_write(0, 0, q35mix.STATE_RECURRENT, f["state"])
            c.state_write(0, 0, q35mix.STATE_CONV, f["conv_state"])
            T = f["qkv"].shape[0]
            args = [c.array(f[k].shape, f[k]) for k in ("qkv", "z", "b", "a")]
            out = c.array((T, c.value_dim))
            if name == "deltanet_decode":
                c.deltanet_decode(0, [0], *args, out)
            else:
                c.deltanet_prefill(0, 0, T, *args, out)
            assert rel(out.download().reshape(f["out"].shape), f["out"]) <= 1e-4
            assert rel(c.state_read(0, 0, q35mix.STATE_RECURRENT), f["state_out"]) <= 1e-4
            np.testing.assert_array_equal(c.state_read(0, 0, q35mix.STATE_CONV),
                                          f["conv_state_out"])
        else:
            c.set_attn_weights(1, f)
            start = f["cache_k"].shape[0]
            c.state_write(1, 0, q35mix.STATE_KEYS, f["cache_k"])
            c.state_write(1, 0, q35mix.STATE_VALUES, f["cache_v"])
            c.advance(0, start)
            T = f["q_gate"].shape[0]
            args = [c.array(f[k].shape, f[k]) for k in ("q_gate", "k", "v")]
            out = c.array((T, c.q_dim))
            if name == "attn_decode":
                c.attn_decode(1, [0], *args, out)
                krow = c.state_read(1, 0, q35mix.STATE_KEYS, rows=start + 1)[start]
                assert rel(krow, f["k_row"]) <= 1e-4
            else:
                c.attn_prefill(1, 0, T, *args, out)
                krows = c.state_read(1, 0, q35mix.STATE_KEYS, rows=start + T)[start:]
                assert rel(krows, f["k_rows"]) <= 1e-4
            assert rel(out.download().reshape(f["out"].shape), f["out"]) <= 1e-4
