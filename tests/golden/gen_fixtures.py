"""Writes the committed golden fixtures of the mixer path (tests/golden/*.npz).

The reference (C# .NET) cannot run in this environment and holds no golden
vectors of its own, so the fixtures are produced by the CPU oracle (the C
restatement of the reference, pinned by tests/test_oracle.py) at the smallest
shapes the HIP kernels accept (dk = dv = 128, head_dim = 256): one k-head with
two v-heads, and one kv head with four q heads.  Inputs come from the seeded
generator in qwen3.5sharp_amd/synth.py.  manifest.json records the SHA-256 of
every file.  Run from the repository root:  python tests/golden/gen_fixtures.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "qwen3.5sharp_amd")]

import oracle  # noqa: E402
import synth  # noqa: E402

NK, NV, HD = 1, 2, 128
NH, NKV, AHD = 4, 1, 256


def cases():
    d = oracle.dims(n_k_heads=NK, n_v_heads=NV, n_heads=NH, n_kv_heads=NKV)
    w = synth.deltanet_weights(NK, NV, HD, salt=7)
    st = synth.deltanet_state(NK, NV, HD, salt=7)
    x = synth.deltanet_inputs(1, NK, NV, HD, salt=8)
    out, cs, s, core = oracle.deltanet_decode(d, x["qkv"][0], x["z"][0], x["b"][0], x["a"][0], w,
                                              st["conv_state"], st["state"])
    yield "deltanet_decode", dict(w, **{k: v for k, v in x.items()}, conv_state=st["conv_state"],
                                  state=st["state"], out=out, conv_state_out=cs, state_out=s)
    for T in (2, 5):
        x = synth.deltanet_inputs(T, NK, NV, HD, salt=9 + T)
        out, cs, s, _ = oracle.deltanet_prefill(d, T, x["qkv"], x["z"], x["b"], x["a"], w,
                                                st["state"], st["conv_state"])
        yield f"deltanet_prefill_T{T}", dict(w, **x, conv_state=st["conv_state"],
                                             state=st["state"], out=out, conv_state_out=cs,
                                             state_out=s)
    wa = synth.attn_weights(AHD, salt=7)
    start = 5
    ck, cv = synth.kv_prefill(start, NKV * AHD, salt=7)
    xa = synth.attn_inputs(1, NH, NKV, AHD, salt=8)
    full_k = np.zeros((start + 1, NKV * AHD), np.float32)
    full_v = np.zeros_like(full_k)
    full_k[:start], full_v[:start] = ck, cv
    out, k2, v2 = oracle.attn_decode(d, start, xa["q_gate"][0], xa["k"][0], xa["v"][0], wa,
                                     full_k, full_v)
    yield "attn_decode", dict(wa, **xa, cache_k=ck, cache_v=cv, out=out, k_row=k2[start])
    T, start = 3, 2
    ck, cv = synth.kv_prefill(start, NKV * AHD, salt=9)
    xa = synth.attn_inputs(T, NH, NKV, AHD, salt=10)
    full_k = np.zeros((start + T, NKV * AHD), np.float32)
    full_v = np.zeros_like(full_k)
    full_k[:start], full_v[:start] = ck, cv
    out, k2, v2 = oracle.attn_prefill(d, start, T, xa["q_gate"], xa["k"], xa["v"], wa, full_k,
                                      full_v)
    yield "attn_prefill", dict(wa, **xa, cache_k=ck, cache_v=cv, out=out, k_rows=k2[start:])


def main():
    manifest = {}
    for name, arrays in cases():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez(path, **{k: np.ascontiguousarray(v, np.float32) for k, v in arrays.items()})
        manifest[f"{name}.npz"] = hashlib.sha256(open(path, "rb").read()).hexdigest()
    manifest["_shapes"] = {"deltanet": {"n_k_heads": NK, "n_v_heads": NV, "head_k_dim": HD},
                           "attention": {"n_heads": NH, "n_kv_heads": NKV, "head_dim": AHD}}
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
