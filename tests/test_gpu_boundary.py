"""The layer boundary (q35m_add_rmsnorm) through the C ABI against the oracle:
bit-exact residual add and zero-centred RMSNorm (the reference's 8 FMA lanes,
horizontal sum, dim % 8 tail, IEEE sqrt and division), at the hidden sizes of
the 4B mixers, tail widths, 1 to 2048 tokens, with and without the residual
and the weight, and the fused Q8_K output byte-identical to q35m_quantize_q8k
of the same y."""
import sys

import numpy as np
import pytest

import oracle
import q35mix

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), n_seqs=1, kv_capacity=16)
    yield c
    c.close()


CASES = [(2560, 1, True, True), (2560, 7, True, False), (4096, 3, False, True), (2560, 2048, True, True),
         (12, 5, True, True), (20, 2, False, False), (256, 9, True, True), (16384, 2, True, True)]


@pytest.mark.parametrize("dim,tokens,add,weighted", CASES)
def test_add_rmsnorm_bit_exact(ctx, dim, tokens, add, weighted):
    say(f"add_rmsnorm dim={dim} tokens={tokens} add={add} weighted={weighted}")
    rng = np.random.default_rng(dim + 7 * tokens)
    h = (rng.standard_normal((tokens, dim)) * rng.uniform(0.05, 20, (tokens, 1))).astype(np.float32)
    d = rng.standard_normal((tokens, dim)).astype(np.float32) if add else None
    w = (rng.standard_normal(dim) * 0.1).astype(np.float32) if weighted else None
    want_h, want_y = oracle.add_rmsnorm(h, d, w, dim, eps=1e-6)
    dh = ctx.array((tokens, dim), h)
    dd = ctx.array((tokens, dim), d) if add else None
    dw = ctx.array((dim,), w) if weighted else None
    dy = ctx.array((tokens, dim))
    q8 = None
    if dim % 256 == 0:
        q8 = q35mix.DeviceBytes(ctx, np.zeros(q35mix.lib().q35m_q8k_bytes(dim, tokens), np.uint8))
    ctx.add_rmsnorm(dh, dd, dw, dy, q8, dim, tokens, 1e-6)
    got_h, got_y = dh.download(), dy.download()
    assert np.array_equal(got_h.view(np.uint32), want_h.view(np.uint32))
    bad = np.flatnonzero(got_y.view(np.uint32) != want_y.view(np.uint32))
    say(f"  y mismatches {bad.size} of {got_y.size}")
    assert bad.size == 0
    if q8 is not None:
        ref = ctx.quantize_q8k(dy, dim, tokens)
        assert np.array_equal(q8.download(), ref.download())
        ref.free()
        q8.free()
    for a in (dh, dd, dw, dy):
        if a is not None:
            a.free()


def test_q8_only_and_in_place(ctx):
    """y NULL with q8 given; y aliasing hidden (the reference's in-place use)."""
    dim, tokens = 2560, 4
    rng = np.random.default_rng(12)
    h = rng.standard_normal((tokens, dim)).astype(np.float32)
    w = (rng.standard_normal(dim) * 0.1).astype(np.float32)
    _, want_y = oracle.add_rmsnorm(h, None, w, dim, eps=1e-6)
    dh, dw = ctx.array((tokens, dim), h), ctx.array((dim,), w)
    q8 = q35mix.DeviceBytes(ctx, np.zeros(q35mix.lib().q35m_q8k_bytes(dim, tokens), np.uint8))
    ctx.add_rmsnorm(dh, None, dw, None, q8, dim, tokens, 1e-6)
    dy = ctx.array((tokens, dim), want_y)
    ref = ctx.quantize_q8k(dy, dim, tokens)
    assert np.array_equal(q8.download(), ref.download())
    ctx.add_rmsnorm(dh, None, dw, dh, None, dim, tokens, 1e-6)
    assert np.array_equal(dh.download().view(np.uint32), want_y.view(np.uint32))
    for a in (dh, dw, q8, dy, ref):
        a.free()


def test_rejects_bad_arguments(ctx):
    L, hnd = q35mix.lib(), ctx.handle
    dh = ctx.array((2, 512))
    assert L.q35m_add_rmsnorm(hnd, dh.ptr, None, None, None, None, 512, 2, 1e-6) == q35mix.ERR_INVALID
    assert L.q35m_add_rmsnorm(hnd, dh.ptr, None, None, dh.ptr, None, 510, 2, 1e-6) == q35mix.ERR_UNSUPPORTED
    assert L.q35m_add_rmsnorm(hnd, dh.ptr, None, None, dh.ptr, dh.ptr, 500, 2, 1e-6) == q35mix.ERR_UNSUPPORTED
    assert L.q35m_add_rmsnorm(hnd, dh.ptr + 4, None, None, dh.ptr, None, 512, 2, 1e-6) == q35mix.ERR_INVALID
    assert L.q35m_add_rmsnorm(hnd, dh.ptr, None, None, dh.ptr, None, 512, 0, 1e-6) == q35mix.ERR_INVALID
    dh.free()
