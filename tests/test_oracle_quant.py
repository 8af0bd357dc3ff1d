"""Pins the oracle's quantized-projection restatement (oracle/q35_oracle_quant.c).

The reference has no tests for Q4_K / Q5_K / Q6_K / Q2_0C / STQ1_0 / Q8_K, so
the restatement is pinned by what the formats and the mathematics fix (IQ4_XS
also by the reference's own IQ4XSTests, ported with the same .NET Random
draws):
  - fp16 decoding against numpy's float16 for every bit pattern;
  - Q8_K: the first extremum maps to exactly -127, ties round to even, the
    sign of the scale follows the first extremum, bsums are the sums of 16,
    and every value reconstructs within half a step;
  - dequantization of every format against independent numpy decoders of
    the bit layouts (Q4_K / Q5_K scales through the per-index GetScaleMin
    formula, not the word-mask unpacking the dot products use; STQ1_0 through
    a reshape of its group / lane order); the STQ1_0 codebook by its
    invariants (one zero lane per pattern, the sign bit negates, all 32
    one-zero ternary patterns present);
  - Q2_0C / STQ1_0 dots exactly equal to the integer dot of the decoded
    values when every scale is 1, and which rows take the panel order;
  - the integer dot products against fp64 dots of the dequantized weights
    with the dequantized activations (equal in exact arithmetic), and exact
    values on hand-built blocks.
The fp32 lane order of the reference's AVX2 accumulation is restated, not
pinned bit for bit (no reference run is possible here).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import oracle  # noqa: E402
import quant_blocks as qb  # noqa: E402
from test_oracle import DotNetRandom  # noqa: E402

ALL_TYPES = [1, 2, 4, 5, 6, 14]


def test_half_to_float_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_q8k_zero_block_and_rules():
    x = np.zeros(512, dtype=np.float32)
    x[256 + 7] = -127.0          # first extremum of block 1, negative -> iscale = 1
    x[256 + 9] = 127.0
    x[256 + 1], x[256 + 2], x[256 + 3], x[256 + 4] = 2.5, 3.5, -2.5, 0.49999997
    d, q, bs = qb.parse_q8k(oracle.q8k_quantize(x))
    assert d[0] == 0 and not q[0].any() and not bs[0].any()
    assert d[1] == 1.0
    assert q[1][7] == -127 and q[1][9] == 127
    assert list(q[1][1:5]) == [2, 4, -2, 0]     # ties to even
    # first extremum positive -> negative scale
    y = np.zeros(256, dtype=np.float32)
    y[3], y[5] = 4.0, -4.0
    d2, q2, _ = qb.parse_q8k(oracle.q8k_quantize(y))
    assert d2[0] < 0 and q2[0][3] == -127 and q2[0][5] == 127


def test_q8k_random_against_numpy():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(256 * 64) * rng.uniform(0.01, 50, 256 * 64)).astype(np.float32)
    d, q, bs = qb.parse_q8k(oracle.q8k_quantize(x))
    xb = x.reshape(64, 256)
    for i in range(64):
        amax = np.abs(xb[i]).max()
        first = int(np.argmax(np.abs(xb[i]) == amax))
        mx = xb[i][first]
        iscale = np.float32(-127.0) / np.float32(mx)
        qq = np.clip(np.rint(xb[i] * iscale), -127, 127).astype(np.int8)
        assert np.array_equal(q[i], qq)
        assert d[i] == np.float32(1.0) / iscale
        assert q[i][first] == -127
        assert np.array_equal(bs[i], q[i].astype(np.int32).reshape(16, 16).sum(1))
        assert np.all(np.abs(xb[i].astype(np.float64) - d[i] * q[i]) <= 0.5 * abs(d[i]) * (1 + 1e-6))


@pytest.mark.parametrize("qtype", ALL_TYPES)
def test_dequantize_against_numpy_decoder(qtype):
    rng = np.random.default_rng(3 + qtype)
    w = qb.random_blocks(rng, qtype, 24)
    got = oracle.dequantize(qtype, w, 24 * qb.VALUES[qtype])
    want = qb.dequant(qtype, w)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("qtype", ALL_TYPES)
def test_dot_against_fp64(qtype):
    rng = np.random.default_rng(20 + qtype)
    n = 256 * 16
    for trial in range(8):
        w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n))
        x = (rng.standard_normal(n) * (1 + 3 * trial)).astype(np.float32)
        q8 = oracle.q8k_quantize(x)
        d, q, _ = qb.parse_q8k(q8)
        xd = (d[:, None].astype(np.float64) * q.astype(np.float64)).ravel()
        wd = qb.dequant_f64(qtype, w)
        exact = float(np.dot(wd, xd))
        scale = float(np.dot(np.abs(wd), np.abs(xd)))
        got = oracle.dot(qtype, w, q8, n)
        assert abs(got - exact) <= 2e-6 * scale + 1e-30, (trial, got, exact)


def test_q4k_dot_hand_built():
    # d = 1, dmin = 0.5, every scale 1, every min 2, every nibble 1 (low) / 3 (high);
    # q8 all 1 with D = 1: sum = 128*1 + 128*3 - 8 sub-blocks * 2 * 0.5 * 32 = 256.
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[4:16] = qb.pack_q4k_scales([1] * 8, [2] * 8)
    blk[16:] = 0x31
    x = np.full(256, -1.0, dtype=np.float32)        # first extremum negative: D = 1/127*...
    x[0] = -127.0
    x[1:] = -127.0                                  # all equal -> q = -127, D = 1
    q8 = oracle.q8k_quantize(x)
    d, q, _ = qb.parse_q8k(q8)
    assert d[0] == 1.0 and np.all(q[0] == -127)
    # dot = -127 * (128*1 + 128*3) - 0.5*2*(-127*256) = -127*512 + 127*256
    assert oracle.q4k_dot(blk, q8, 256) == np.float32(-127 * 512 + 127 * 256)


def test_q6k_dot_hand_built():
    # d = 0.25, scales alternate 2 / -1, every 6-bit value 40 (-> 8 after the -32)
    blk = np.zeros(210, dtype=np.uint8)
    vals = np.full(256, 40, dtype=np.int64)
    blk[:192] = qb.pack_q6k_values(vals)
    blk[192:208] = np.array([2, -1] * 8, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    x = np.full(256, -127.0, dtype=np.float32)
    q8 = oracle.q8k_quantize(x)
    # sum over 16 sub-blocks of 16 values: scale * 8 * (-127); 8 sub-blocks at 2, 8 at -1
    want = 0.25 * 16 * 8 * (-127) * (8 * 2 + 8 * -1)
    assert oracle.q6k_dot(blk, q8, 256) == np.float32(want)


def test_q5k_dot_hand_built():
    # d = 1, dmin = 0.5, every scale 1, every min 2, every nibble 1 (low) / 3
    # (high), every qh bit set (+16): values 17 and 19; q8 all -127 with D = 1:
    # -127 * 128 * (17 + 19) - 0.5 * (16 * 16 * -127 * 2).
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[4:16] = qb.pack_q4k_scales([1] * 8, [2] * 8)
    blk[16:48] = 0xFF
    blk[48:] = 0x31
    q8 = oracle.q8k_quantize(np.full(256, -127.0, dtype=np.float32))
    want = -127 * 128 * 36 - 0.5 * (16 * 16 * -127 * 2)
    assert oracle.q5k_dot(blk, q8, 256) == np.float32(want)
    # the high bit matters: clearing qh gives values 1 and 3
    blk[16:48] = 0
    assert oracle.q5k_dot(blk, q8, 256) == np.float32(-127 * 128 * 4 - 0.5 * (16 * 16 * -127 * 2))


def test_iq4xs_dot_hand_built():
    # d = 1, every sub-block scale ls = 33 (dl = 1: low nibble 1, high bits 2),
    # every byte 0x8F (low nibble 15 -> 113, high nibble 8 -> 1); q8 all -127,
    # D = 1: 8 sub-blocks of -127 * 16 * (113 + 1).
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.uint16(0xAAAA).tobytes(), np.uint8)
    blk[4:8] = 0x11
    blk[8:] = 0x8F
    q8 = oracle.q8k_quantize(np.full(256, -127.0, dtype=np.float32))
    assert oracle.iq4xs_dot(blk, q8, 256) == np.float32(8 * -127 * 16 * 114)
    # sub-block scale ls = 31 on sub-block 0 only (dl = -1): scales_l low nibble 15, high bits 1
    blk[4] = 0x1F
    blk[2:4] = np.frombuffer(np.uint16(0xAAA9).tobytes(), np.uint8)
    assert oracle.iq4xs_dot(blk, q8, 256) == np.float32(6 * -127 * 16 * 114)


def _force_valid_scales(raw, nb):
    """IQ4XSTests.ForceValidScales: every block's fp16 grid scale = 1.0."""
    for i in range(nb):
        raw[i * 136] = 0x00
        raw[i * 136 + 1] = 0x3C


def test_iq4xs_reference_dequantize_row():
    """Port of IQ4XSTests.DequantizeRow_MatchesReference
    (tests/Qwen35Sharp.Tests/IQ4XSTests.cs:13-53): Random(7) bytes for 3
    super-blocks, scales forced to 1.0, against the llama.cpp formula, 1e-4."""
    nb, k = 3, 768
    rng = DotNetRandom(7)
    raw = bytearray(rng.next_bytes(nb * 136))
    _force_valid_scales(raw, nb)
    raw = np.frombuffer(bytes(raw), np.uint8)
    expected = np.zeros(k, np.float32)
    grid = qb.IQ4_GRID
    for i in range(nb):
        blk = raw[i * 136:(i + 1) * 136]
        d = np.float32(blk[0:2].copy().view(np.float16)[0])
        sh = int(blk[2:4].copy().view(np.uint16)[0])
        qs = blk[8:]
        for ib in range(8):
            ls = ((int(blk[4 + ib // 2]) >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)
            dl = np.float32(d * np.float32(ls - 32))
            for j in range(16):
                expected[i * 256 + ib * 32 + j] = dl * np.float32(grid[qs[16 * ib + j] & 0xF])
                expected[i * 256 + ib * 32 + j + 16] = dl * np.float32(grid[qs[16 * ib + j] >> 4])
    got = oracle.dequantize(14, raw, k)
    assert np.all(np.abs(expected - got) < 1e-4)


def test_iq4xs_reference_dot():
    """Port of IQ4XSTests.Dot_MatchesScalarDequant (IQ4XSTests.cs:55-101):
    Random(9) bytes for 2 super-blocks, scales forced to 1.0, activations
    NextDouble() * 4 - 2 quantized to Q8_K; the dot against the fp32 sum of
    the dequantized products, within 1e-2 or 1e-4 relative."""
    nb, k = 2, 512
    rng = DotNetRandom(9)
    raw = bytearray(rng.next_bytes(nb * 136))
    _force_valid_scales(raw, nb)
    raw = np.frombuffer(bytes(raw), np.uint8)
    act = np.array([np.float32(rng.next_double() * 4 - 2) for _ in range(k)], np.float32)
    q8 = oracle.q8k_quantize(act)
    dot = oracle.iq4xs_dot(raw, q8, k)
    iq = oracle.dequantize(14, raw, k)
    d, q, _ = qb.parse_q8k(q8)
    q8v = (d[:, None] * q.astype(np.float32)).astype(np.float32).ravel()
    expected = np.float32(0)
    for i in range(k):
        expected = np.float32(expected + np.float32(iq[i] * q8v[i]))
    err = abs(float(expected) - float(dot))
    assert err < 1e-2 or err < 1e-4 * abs(float(expected)), (expected, dot)


@pytest.mark.parametrize("qtype", ALL_TYPES)
def test_linear_q_against_fp64(qtype):
    rng = np.random.default_rng(40 + qtype)
    n_in, n_out, tokens = 512, 96, 3
    w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
    x = rng.standard_normal((tokens, n_in)).astype(np.float32)
    y = oracle.linear_q(qtype, w, x, n_in, n_out)
    wd = qb.dequant_f64(qtype, w).reshape(n_out, n_in)
    for t in range(tokens):
        d, q, _ = qb.parse_q8k(oracle.q8k_quantize(x[t]))
        xd = (d[:, None].astype(np.float64) * q).ravel()
        exact = wd @ xd
        scale = np.abs(wd) @ np.abs(xd)
        assert np.all(np.abs(y[t] - exact) <= 2e-6 * scale)


def test_q4k_several_tokens_panel_rows_and_gemv_tail():
    """Several tokens: the first n_out & ~7 outputs follow the panel GEMM order,
    the rest the GEMV; one token is the GEMV throughout.  All within fp32
    rounding of the exact value, and the two orders really differ."""
    rng = np.random.default_rng(91)
    n_in, n_out = 1024, 13
    w = qb.random_blocks(rng, 4, n_out * n_in // 256)
    x = rng.standard_normal((3, n_in)).astype(np.float32)
    y = oracle.linear_q(4, w, x, n_in, n_out)
    wd = qb.dequant_f64(4, w).reshape(n_out, n_in)
    rows = w.reshape(n_out, -1)
    differ = 0
    for t in range(3):
        q8 = oracle.q8k_quantize(x[t])
        gemv = np.array([oracle.q4k_dot(rows[r], q8, n_in) for r in range(n_out)], np.float32)
        assert np.array_equal(y[t, 8:].view(np.uint32), gemv[8:].view(np.uint32))
        differ += int(np.sum(y[t, :8].view(np.uint32) != gemv[:8].view(np.uint32)))
        d, q, _ = qb.parse_q8k(q8)
        xd = (d[:, None].astype(np.float64) * q).ravel()
        assert np.all(np.abs(y[t] - wd @ xd) <= 2e-6 * (np.abs(wd) @ np.abs(xd)))
    assert differ > 0
    y1 = oracle.linear_q(4, w, x[:1], n_in, n_out)
    q8 = oracle.q8k_quantize(x[0])
    gemv = np.array([oracle.q4k_dot(rows[r], q8, n_in) for r in range(n_out)], np.float32)
    assert np.array_equal(y1[0].view(np.uint32), gemv.view(np.uint32))


def test_stq_codebook_invariants():
    cb = qb.STQ_CODEBOOK.astype(np.int64)
    lanes = np.stack([(cb >> (2 * l)) & 3 for l in range(4)], axis=1) - 1      # [32][4]
    assert np.all(np.sum(lanes == 0, axis=1) == 1)                              # one zero lane
    assert np.all(np.isin(lanes, [-1, 0, 1]))
    assert np.array_equal(lanes[16:], -lanes[:16])                              # sign bit negates
    pats = {tuple(r) for r in lanes}
    want = {tuple(np.insert(np.array(sg), z, 0)) for z in range(4)
            for sg in np.array(np.meshgrid([-1, 1], [-1, 1], [-1, 1])).T.reshape(-1, 3)}
    assert pats == want and len(pats) == 32
    # the oracle's table is the same one: slot s with sign 0 / 1 decodes to lanes[s] / lanes[16 + s]
    for sign in (0, 1):
        blk = np.zeros(42, np.uint8)
        blk[0:32] = np.arange(64, dtype=np.uint8)[0::2] % 16 | ((np.arange(64, dtype=np.uint8)[1::2] % 16) << 4)
        blk[32:40] = 0xFF * sign
        blk[40:42] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        vals = oracle.dequantize(1, blk, 256).astype(np.int64)
        for g in range(64):
            chunk, gloc = g >> 4, g & 15
            got = [vals[chunk * 64 + gloc + 16 * l] for l in range(4)]
            assert got == list(lanes[16 * sign + g % 16]), (sign, g)


def _unit_scale_blocks(rng, qtype, nb):
    w = qb.random_blocks(rng, qtype, nb).reshape(nb, qb.BYTES[qtype])
    d_off = 40 if qtype == 1 else 0
    w[:, d_off:d_off + 2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    return w.ravel()


@pytest.mark.parametrize("qtype", [1, 2])
def test_ternary_dots_exact_with_unit_scales(qtype):
    """Unit weight scales and a Q8_K scale of 1 (every block's first extremum
    -127): the dot is the exact integer dot of the decoded values with the
    int8 activations, in both orders (raw dot, and the panel rows of a call)."""
    rng = np.random.default_rng(70 + qtype)
    n = 2048
    for trial in range(6):
        w = _unit_scale_blocks(rng, qtype, qb.nblocks(qtype, n))
        x = rng.integers(-127, 128, n).astype(np.float32)
        x[::256] = -127.0
        q8 = oracle.q8k_quantize(x)
        d, q, _ = qb.parse_q8k(q8)
        assert np.all(d == 1.0) and np.array_equal(q.ravel(), x.astype(np.int8))
        vals = np.concatenate([qb.stq_values(b) if qtype == 1 else qb.q2_values(b)
                               for b in w.reshape(-1, qb.BYTES[qtype])])
        exact = int(np.dot(vals, x.astype(np.int64)))
        assert oracle.dot(qtype, w, q8, n) == np.float32(exact)
        y = oracle.linear_q(qtype, np.tile(w, 8), x[None, :], n, 8)       # eight panel rows
        assert np.all(y == np.float32(exact))


def _raw_rows(qtype, w, x, n_in, n_out):
    rows = w.reshape(n_out, -1)
    out = np.empty((x.shape[0], n_out), np.float32)
    for t in range(x.shape[0]):
        q8 = oracle.q8k_quantize(x[t])
        out[t] = [oracle.dot(qtype, rows[r], q8, n_in) for r in range(n_out)]
    return out


@pytest.mark.parametrize("qtype,tokens,n_out,panel_rows", [
    (2, 1, 13, 8), (2, 3, 13, 8), (2, 5, 16, 16), (2, 2, 5, 0),
    (1, 1, 13, 8), (1, 3, 16, 0), (1, 4, 16, 16), (1, 4, 13, 0), (1, 8, 24, 24), (1, 2, 7, 0)])
def test_ternary_panel_rows(qtype, tokens, n_out, panel_rows):
    """Which rows take the eight-row panel order: Q2_0C the first n_out & ~7
    for any token count; STQ1_0 the same for one token, and for several all
    rows when tokens % 4 == 0 and n_out % 8 == 0, else none.  The other rows
    equal the raw-row dot; panel rows differ from it somewhere; all are within
    fp32 rounding of the exact value."""
    rng = np.random.default_rng(100 * qtype + 10 * tokens + n_out)
    n_in = 4096
    w = qb.random_blocks(rng, qtype, qb.nblocks(qtype, n_out * n_in))
    x = rng.standard_normal((tokens, n_in)).astype(np.float32)
    y = oracle.linear_q(qtype, w, x, n_in, n_out)
    raw = _raw_rows(qtype, w, x, n_in, n_out)
    assert np.array_equal(y[:, panel_rows:].view(np.uint32), raw[:, panel_rows:].view(np.uint32))
    if panel_rows:
        assert np.any(y[:, :panel_rows].view(np.uint32) != raw[:, :panel_rows].view(np.uint32))
    wd = qb.dequant_f64(qtype, w).reshape(n_out, n_in)
    for t in range(tokens):
        d, q, _ = qb.parse_q8k(oracle.q8k_quantize(x[t]))
        xd = (d[:, None].astype(np.float64) * q).ravel()
        assert np.all(np.abs(y[t] - wd @ xd) <= 2e-6 * (np.abs(wd) @ np.abs(xd)))


def test_q2_dot_hand_built():
    # d = 0.5; half 0 codes 3 (+3), half 1 codes 1 (-1); activations -127 with
    # Q8_K scale 1 in block 0 and -63.5 (scale 0.5) in block 1:
    # 0.5 * (3 * -127 * 256 * 1 + -1 * -127 * 256 * 0.5)
    blk = np.zeros(130, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:66] = 0xFF
    blk[66:130] = 0x55
    x = np.concatenate([np.full(256, -127.0), np.full(256, -63.5)]).astype(np.float32)
    q8 = oracle.q8k_quantize(x)
    want = 0.5 * (3 * -127 * 256 + -1 * -127 * 256 * 0.5)
    assert oracle.q2_0c_dot(blk, q8, 512) == np.float32(want)
    assert oracle.linear_q(2, np.tile(blk, 8), x[None, :], 512, 8)[0, 3] == np.float32(want)


def test_stq_dot_hand_built():
    # slot 0, sign 0: lanes (0, +1, +1, +1) -> the first 16 values of every
    # 64-value chunk are 0, the other 48 are +1; sign 1 negates.  d = 0.25,
    # activations -127 (Q8_K scale 1): 0.25 * 4 * 48 * -127 per block.
    blk = np.zeros(42, np.uint8)
    blk[40:42] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    q8 = oracle.q8k_quantize(np.full(256, -127.0, np.float32))
    assert oracle.stq1_0_dot(blk, q8, 256) == np.float32(0.25 * 4 * 48 * -127)
    blk[32:40] = 0xFF
    assert oracle.stq1_0_dot(blk, q8, 256) == np.float32(-0.25 * 4 * 48 * -127)
    # activations nonzero only on the first 16 of each chunk: the zero lane
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    for c in range(4):
        x[64 * c + 1:64 * c + 16] = 5.0
    assert oracle.stq1_0_dot(blk, oracle.q8k_quantize(x), 256) == 0.0


def test_linear_f32_lane_order():
    """Ops.DotF32's order, pinned on rows whose sum depends on it: 2^24 in
    lane 0 and ones elsewhere.  With 17 elements the 16 lanes hold 2^24, 1 x 15
    (2^24 + 1 rounds back to 2^24 in acc0 + acc1), the horizontal sum gives
    2^24 + 14, and the scalar tail adds 1 more: 2^24 + 15 rounds to 2^24 + 16.
    A sequential sum would stay at 2^24.  With 24 elements the 8-wide chunk
    goes into acc0 (lane 0 gets 2^24 + 1 -> 2^24 again)."""
    big = np.float32(2.0 ** 24)
    for n, want in ((17, 2.0 ** 24 + 16), (24, 2.0 ** 24 + 22), (7, 2.0 ** 24)):
        x = np.ones((1, n), np.float32)
        x[0, 0] = big
        w = np.ones((1, n), np.float32)
        got = oracle.linear_f32(w, x, n, 1)[0, 0]
        assert got == np.float32(want), (n, got)


def test_linear_f32_against_fp64():
    rng = np.random.default_rng(123)
    for n_in, n_out, tokens in ((2560, 32, 2), (31, 5, 3), (8, 4, 1), (4099, 9, 2)):
        w = rng.standard_normal((n_out, n_in)).astype(np.float32)
        x = rng.standard_normal((tokens, n_in)).astype(np.float32)
        y = oracle.linear_f32(w, x, n_in, n_out)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        scale = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
        assert np.all(np.abs(y - exact) <= 2e-6 * scale)
