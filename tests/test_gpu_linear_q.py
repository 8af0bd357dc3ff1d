"""Quantized projections (q35m_linear_q4k / _q5k / _q6k / _iq4xs / _q2_0c /
_stq1_0) through the C ABI against the oracle: bit-exact (the kernels keep the
reference's integer lanes and fp32 accumulation order: the AVX2 GEMV for one
token and for Q6_K, the panel GEMM for Q4_K with several tokens plus the GEMV
for its last n_out % 8 outputs, the scalar per-token dot of Q5_K and IQ4_XS,
the eight-row panel and raw-row orders of Q2_0C and STQ1_0 split as the
reference splits them, by row and, for STQ1_0, by token count), at the
projection shapes of the 4B mixers
(hidden 2560: qkv 8192, gate 4096, beta/alpha 32, ssm_out and attn_output
4096 -> 2560, attn k/v 1024), ragged small shapes, several tokens, zero and
extreme activation blocks, and weight buffers whose size is not a multiple of
16 bytes."""
import sys

import numpy as np
import pytest

import oracle
import q35mix
import quant_blocks as qb

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), n_seqs=1,
                       kv_capacity=16)
    yield c
    c.close()


def run(ctx, qtype, w, x, n_in, n_out):
    tokens = x.shape[0]
    dw = ctx.bytes_array(w)
    dx = ctx.array((tokens, n_in), x)
    dy = ctx.array((tokens, n_out))
    ctx.linear_q(qtype, dw, dx, dy, n_in, n_out, tokens)
    y = dy.download()
    for a in (dw, dx, dy):
        a.free()
    return y


SHAPES = [(2560, 8192, 1), (2560, 4096, 1), (2560, 32, 1), (4096, 2560, 1), (2560, 1024, 1),
          (256, 7, 1), (512, 33, 5), (2560, 1024, 3), (16384, 19, 2), (2560, 520, 70),
          (4096, 136, 130), (512, 40, 16), (1024, 72, 15), (2560, 64, 4), (1024, 13, 4), (1536, 24, 8),
          (768, 33, 20), (768, 40, 20)]


NAMES = {1: "STQ1_0", 2: "Q2_0C", 4: "Q4_K", 5: "Q5_K", 6: "Q6_K", 14: "IQ4_XS"}
TYPES = [1, 2, 4, 5, 6, 14]


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n_in,n_out,tokens", SHAPES)
def test_linear_q_bit_exact(ctx, qtype, n_in, n_out, tokens):
    if n_in % qb.VALUES[qtype]:
        n_in += qb.VALUES[qtype] - n_in % qb.VALUES[qtype]
    say(f"linear_q {NAMES[qtype]} n_in={n_in} n_out={n_out} tokens={tokens}")
    rng = np.random.default_rng(1000 * qtype + n_in + n_out + tokens)
    w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
    x = rng.standard_normal((tokens, n_in)).astype(np.float32)
    got = run(ctx, qtype, w, x, n_in, n_out)
    want = oracle.linear_q(qtype, w, x, n_in, n_out)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    say(f"  mismatches {bad.size} of {got.size}; max|d| {np.max(np.abs(got - want)):.3e}")
    assert bad.size == 0


@pytest.mark.parametrize("qtype", TYPES)
def test_linear_q_activation_edges(ctx, qtype):
    """Zero blocks (scale 0), a first extremum that is positive (negative
    scale) or repeated with both signs, ties at .5 after scaling, huge and tiny
    magnitudes, and an fp16 subnormal weight scale."""
    n_in, n_out = 2048, 40
    rng = np.random.default_rng(77 + qtype)
    w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
    d_off = {6: 208, 1: 40}.get(qtype, 0)
    w.reshape(-1, qb.BYTES[qtype])[3, d_off:d_off + 2] = np.frombuffer(np.float16(3e-6).tobytes(), np.uint8)
    x = rng.standard_normal((2, n_in)).astype(np.float32)
    x[0, 0:256] = 0.0
    x[0, 256:512] *= 1e-30
    x[0, 512 + 5], x[0, 512 + 9] = 50.0, -50.0
    x[0, 768 + 2], x[0, 768 + 1] = 50.0, -50.0
    blk = x[1, 1024:1280]
    blk[:] = np.arange(256, dtype=np.float32) - 128.0   # iscale exactly 127/128... ties
    blk[0] = -127.0
    blk[1:] = np.clip(blk[1:], -126.5, 126.5)
    x[1, 1280:1536] *= 1e20
    got = run(ctx, qtype, w, x, n_in, n_out)
    want = oracle.linear_q(qtype, w, x, n_in, n_out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_linear_q_rejects_bad_arguments(ctx):
    dw = ctx.bytes_array(np.zeros(144 * 4, np.uint8))
    dx = ctx.array((1, 512))
    dy = ctx.array((1, 2))
    L = q35mix.lib()
    h = ctx.handle
    assert L.q35m_linear_q4k(h, dw.ptr, dx.ptr, dy.ptr, 300, 2, 1) == q35mix.ERR_UNSUPPORTED
    assert L.q35m_linear_q4k(h, dw.ptr + 4, dx.ptr, dy.ptr, 512, 2, 1) == q35mix.ERR_INVALID
    assert L.q35m_linear_q6k(h, dw.ptr, dx.ptr, dy.ptr, 512, 0, 1) == q35mix.ERR_INVALID
    assert L.q35m_linear_q6k(h, dw.ptr, dx.ptr, dy.ptr, 512, 2, 0) == q35mix.ERR_INVALID
    assert L.q35m_linear_q6k(h, None, dx.ptr, dy.ptr, 512, 2, 1) == q35mix.ERR_INVALID
    assert L.q35m_linear_q2_0c(h, dw.ptr, dx.ptr, dy.ptr, 256, 2, 1) == q35mix.ERR_UNSUPPORTED
    assert L.q35m_linear_q2_0c_prequant(h, dw.ptr, dx.ptr, dy.ptr, 768, 2, 1) == q35mix.ERR_UNSUPPORTED
    assert L.q35m_linear_stq1_0(h, dw.ptr + 2, dx.ptr, dy.ptr, 512, 2, 1) == q35mix.ERR_INVALID
    for a in (dw, dx, dy):
        a.free()


def test_prequant_matches_one_shot(ctx):
    """Quantize once, three projections (the reference's attention decode:
    Qwen35Model.Decode.cs:286-292), each bit-identical to the one-shot call
    and to the oracle."""
    n_in = 2560
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, n_in)).astype(np.float32)
    dx = ctx.array((2, n_in), x)
    q8 = ctx.quantize_q8k(dx, n_in, 2)
    for qtype, n_out in ((4, 8192), (4, 1024), (6, 1024), (5, 1024), (14, 32), (2, 1024), (1, 8192), (1, 13)):
        w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
        dw = ctx.bytes_array(w)
        dy = ctx.array((2, n_out))
        ctx.linear_q_prequant(qtype, dw, q8, dy, n_in, n_out, 2)
        got = dy.download()
        want = oracle.linear_q(qtype, w, x, n_in, n_out)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (qtype, n_out)
        assert np.array_equal(got.view(np.uint32), run(ctx, qtype, w, x, n_in, n_out).view(np.uint32))
        dw.free()
        dy.free()
    q8.free()
    dx.free()


@pytest.mark.parametrize("n_in,n_out,tokens", [(2560, 32, 1), (2560, 4096, 2), (4096, 129, 3), (17, 70, 5),
                                               (24, 3, 1), (7, 65, 2), (2561, 40, 70), (1, 1, 1)])
def test_linear_f32_bit_exact(ctx, n_in, n_out, tokens):
    """F32 weights: Ops.DotF32's lane order, bit for bit, also at widths that
    are not multiples of 16, 8 or 4 (the scalar loads and the 8-wide stride)."""
    say(f"linear_f32 n_in={n_in} n_out={n_out} tokens={tokens}")
    rng = np.random.default_rng(n_in + 7 * n_out + tokens)
    w = rng.standard_normal((n_out, n_in)).astype(np.float32)
    x = rng.standard_normal((tokens, n_in)).astype(np.float32)
    if n_in >= 17:
        x[0, 0] = 2.0 ** 24          # order-dependent row
        w[0, :] = 1.0
        x[0, 1:] = 1.0
    dw, dx, dy = ctx.array((n_out, n_in), w), ctx.array((tokens, n_in), x), ctx.array((tokens, n_out))
    ctx.linear_f32(dw, dx, dy, n_in, n_out, tokens)
    got = dy.download()
    want = oracle.linear_f32(w, x, n_in, n_out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for a in (dw, dx, dy):
        a.free()


@pytest.mark.parametrize("qtype", [4, 6])
def test_tiled_pieces_match_whole_launch(monkeypatch, qtype):
    """The tiled Q4_K / Q6_K kernels go in pieces of whole row and token tiles
    when a call holds more than 2 GiB of weight rows or activations; a context
    created with a 256 KiB piece limit splits ordinary shapes the same way
    (several row and token pieces here), and the results stay bit-identical to
    the oracle."""
    monkeypatch.setenv("Q35M_TILE_LIMIT_BYTES", str(256 * 1024))
    c = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), n_seqs=1, kv_capacity=16)
    try:
        n_in, n_out, tokens = (2560, 520, 200) if qtype == 4 else (2560, 424, 200)
        say(f"pieces {NAMES[qtype]} n_in={n_in} n_out={n_out} tokens={tokens}")
        rng = np.random.default_rng(4242 + qtype)
        w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
        x = rng.standard_normal((tokens, n_in)).astype(np.float32)
        got = run(c, qtype, w, x, n_in, n_out)
        want = oracle.linear_q(qtype, w, x, n_in, n_out)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        c.close()


BLOCK_SHAPES = [(2560, 8192, 2048), (4096, 2560, 2048), (2560, 520, 70), (512, 33, 5), (4096, 136, 130),
                (16384, 19, 2), (1024, 72, 16), (2560, 1024, 3), (256, 7, 129)]


@pytest.mark.parametrize("qtype", [4, 6])
@pytest.mark.parametrize("n_in,n_out,tokens", BLOCK_SHAPES)
def test_linear_q_block_order(ctx, qtype, n_in, n_out, tokens):
    """q35m_set_projection_order(PROJ_BLOCK): Q6_K from 16 tokens (n_out *
    n_in / 256 even) accumulates each block's exact integer sum and applies
    its fp32 scales once.  Checked against the exact value of the quantized
    product (fp64 of the dequantized weights and Q8_K activations: |y - exact|
    <= 2e-6 sum |w x|, the bound the reference's own order meets) and against
    the oracle's reference order (max|d| / max|ref| <= 1e-4); Q4_K and the
    shapes outside the block-order condition stay bit-identical to the
    reference order."""
    say(f"linear_q block order {NAMES[qtype]} n_in={n_in} n_out={n_out} tokens={tokens}")
    rng = np.random.default_rng(7000 + 1000 * qtype + n_in + n_out + tokens)
    w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
    x = rng.standard_normal((tokens, n_in)).astype(np.float32)
    ctx.set_projection_order(q35mix.PROJ_BLOCK)
    try:
        got = run(ctx, qtype, w, x, n_in, n_out)
    finally:
        ctx.set_projection_order(q35mix.PROJ_REFERENCE)
    blocked = qtype == 6 and tokens >= 16 and (n_out * n_in // 256) % 2 == 0
    check_rows = min(tokens, 24)
    sel = np.unique(np.linspace(0, tokens - 1, check_rows).astype(int))
    want = oracle.linear_q(qtype, w, x[sel], n_in, n_out)
    if not blocked:
        assert np.array_equal(got[sel].view(np.uint32), want.view(np.uint32))
        return
    e = float(np.max(np.abs(got[sel] - want)) / np.max(np.abs(want)))
    wd = qb.dequant_f64(qtype, w).reshape(n_out, n_in)
    worst = 0.0
    for i, t in enumerate(sel):
        d, q, _ = qb.parse_q8k(oracle.q8k_quantize(x[t]))
        xd = (d[:, None].astype(np.float64) * q).ravel()
        exact = wd @ xd
        scale = np.abs(wd) @ np.abs(xd)
        worst = max(worst, float(np.max(np.abs(got[t] - exact) / scale)))
    say(f"  vs reference order {e:.2e}; worst |y - exact| / sum|w x| {worst:.2e}")
    assert e <= 1e-4
    assert worst <= 2e-6
