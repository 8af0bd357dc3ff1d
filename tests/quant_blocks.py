"""numpy helpers for the GGUF Q4_K / Q5_K / Q6_K / IQ4_XS / Q2_0C / STQ1_0 /
Q8_K block formats used by the quantized-projection tests: random blocks,
independent decoders and packers.  Type codes: 1 = STQ1_0, 2 = Q2_0C,
4 = Q4_K, 5 = Q5_K, 6 = Q6_K, 14 = IQ4_XS.

Layouts (src/Qwen35Sharp.Kernels/BlockLayout.cs:32-101 of the reference):
  Q4_K (144 B): f16 d, f16 dmin, u8 scales[12], u8 qs[128]
  Q5_K (176 B): f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
  Q6_K (210 B): u8 ql[128], u8 qh[64], i8 scales[16], f16 d
  IQ4_XS (136 B): f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]
  Q2_0C (130 B, 512 values): f16 d, u8 qs[128] (value 2 code - 3, 4 a byte)
  STQ1_0 (42 B): u8 qs[32] (4-bit codebook slots), u8 sign[8], f16 d
  Q8_K (292 B): f32 d, i8 qs[256], i16 bsums[16]
"""
from __future__ import annotations

import numpy as np

QK = 256
BYTES = {1: 42, 2: 130, 4: 144, 5: 176, 6: 210, 14: 136}
VALUES = {1: 256, 2: 512, 4: 256, 5: 256, 6: 256, 14: 256}     # values per block
# STQ1_0's four-lane patterns, entry 16 sign + slot, two bits a lane
# (0 = -1, 1 = 0, 2 = +1): the format's table (STQ1_0.cs:50-56).
STQ_CODEBOOK = np.array([0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12,
                         0x6A, 0x62, 0x4A, 0x42, 0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4,
                         0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68], dtype=np.uint8)


def nblocks(qtype, n_values):
    return n_values // VALUES[qtype]
# The IQ4_XS grid (llama.cpp kvalues_iq4nl), as the GGUF format defines it.
IQ4_GRID = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int64)


def parse_q8k(buf):
    b = np.asarray(buf, dtype=np.uint8).reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    q = b[:, 4:260].copy().view(np.int8)
    bs = b[:, 260:292].copy().view(np.int16)
    return d, q, bs


def _f16(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def random_blocks(rng, qtype, nblocks, dscale=0.02):
    """Random but well-formed blocks: finite positive fp16 scales of a realistic
    size, every other byte uniform."""
    n = BYTES[qtype]
    b = rng.integers(0, 256, size=(nblocks, n), dtype=np.uint8)
    d = (rng.uniform(0.2, 1.0, nblocks) * dscale).astype(np.float16)
    if qtype in (4, 5):
        b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        dm = (rng.uniform(0.2, 1.0, nblocks) * dscale).astype(np.float16)
        b[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    elif qtype == 14:
        b[:, 0:2] = (d * np.float16(0.05)).view(np.uint8).reshape(-1, 2)   # dl = d (ls - 32), ls < 64
    elif qtype == 2:
        b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    elif qtype == 1:
        b[:, 40:42] = d.view(np.uint8).reshape(-1, 2)
    else:
        b[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return b.ravel()


def q4k_scale_min(sc: np.ndarray, j: int):
    """Q4K.GetScaleMin (src/Qwen35Sharp.Kernels/Q4K.cs:7-18)."""
    if j < 4:
        return int(sc[j] & 63), int(sc[j + 4] & 63)
    return (int((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)),
            int((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)))


def pack_q4k_scales(scales, mins):
    p = np.zeros(12, dtype=np.uint8)
    for g in range(8):
        ls, lm = scales[g], mins[g]
        if g < 4:
            p[g] |= ls
            p[g + 4] |= lm
        else:
            p[g + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            p[g - 4] |= (ls >> 4) << 6
            p[g] |= (lm >> 4) << 6
    return p


def pack_q6k_values(vals):
    """ql[128] | qh[64] for 256 six-bit values (the inverse of the decoder below)."""
    ql = np.zeros(128, dtype=np.uint8)
    qh = np.zeros(64, dtype=np.uint8)
    v = np.asarray(vals, dtype=np.int64)
    for half in range(2):
        base = 128 * half
        for l in range(32):
            q1, q2, q3, q4 = v[base + l], v[base + l + 32], v[base + l + 64], v[base + l + 96]
            ql[64 * half + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * half + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * half + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return np.concatenate([ql, qh])


def stq_values(blk):
    """The 256 ternary values of one STQ1_0 block: group g = 16 chunk + gloc
    (slot: nibble g % 2 of qs[g / 2]; sign: bit g % 8 of sign[g / 8]) holds
    the values at chunk * 64 + gloc + 16 lane, lane = 0..3."""
    qs, sg = blk[0:32], blk[32:40]
    slots = np.stack([qs & 15, qs >> 4], axis=1).ravel().astype(np.int64)          # [64]
    signs = np.unpackbits(sg, bitorder="little").astype(np.int64)                   # [64]
    pat = STQ_CODEBOOK[16 * signs + slots].astype(np.int64)
    lanes = np.stack([(pat >> (2 * l)) & 3 for l in range(4)], axis=1) - 1          # [64 groups][4 lanes]
    return lanes.reshape(4, 16, 4).transpose(0, 2, 1).reshape(256)                  # [chunk][lane][gloc]


def q2_values(blk):
    """The 512 values 2 code - 3 of one Q2_0C block (4 codes a byte, low first)."""
    qs = blk[2:130].astype(np.int64)
    codes = np.stack([(qs >> (2 * k)) & 3 for k in range(4)], axis=1).ravel()
    return 2 * codes - 3


def _dequant(qtype, w, dtype):
    b = np.asarray(w, dtype=np.uint8).reshape(-1, BYTES[qtype])
    out = np.empty((b.shape[0], VALUES[qtype]), dtype=dtype)
    for i, blk in enumerate(b):
        if qtype in (1, 2):
            d = dtype(blk[40:42].copy().view(np.float16)[0] if qtype == 1 else blk[0:2].copy().view(np.float16)[0])
            vals = stq_values(blk) if qtype == 1 else q2_values(blk)
            out[i] = vals.astype(dtype) * d
            continue
        if qtype == 5:
            # llama.cpp dequantize_row_q5_K: 64-value groups j, scale/min pair
            # 2j (low nibbles, qh bit 2j) and 2j + 1 (high nibbles, qh bit 2j + 1)
            d = dtype(blk[0:2].copy().view(np.float16)[0])
            dmin = dtype(blk[2:4].copy().view(np.float16)[0])
            sc, qh, qs = blk[4:16], blk[16:48].astype(np.int64), blk[48:176].astype(np.int64)
            for j in range(4):
                s0, m0 = q4k_scale_min(sc, 2 * j)
                s1, m1 = q4k_scale_min(sc, 2 * j + 1)
                q = qs[32 * j:32 * j + 32]
                lo = (q & 15) + 16 * ((qh >> (2 * j)) & 1)
                hi = (q >> 4) + 16 * ((qh >> (2 * j + 1)) & 1)
                out[i, 64 * j:64 * j + 32] = dtype(d * dtype(s0)) * lo.astype(dtype) - dtype(dmin * dtype(m0))
                out[i, 64 * j + 32:64 * j + 64] = dtype(d * dtype(s1)) * hi.astype(dtype) - dtype(dmin * dtype(m1))
            continue
        if qtype == 14:
            # llama.cpp dequantize_row_iq4_xs
            d = dtype(blk[0:2].copy().view(np.float16)[0])
            sh = int(blk[2:4].copy().view(np.uint16)[0])
            sl, qs = blk[4:8], blk[8:136].astype(np.int64)
            for ib in range(8):
                ls = ((int(sl[ib // 2]) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
                dl = dtype(d * dtype(ls - 32))
                q = qs[16 * ib:16 * ib + 16]
                out[i, 32 * ib:32 * ib + 16] = dl * IQ4_GRID[q & 15].astype(dtype)
                out[i, 32 * ib + 16:32 * ib + 32] = dl * IQ4_GRID[q >> 4].astype(dtype)
            continue
        if qtype == 4:
            d = dtype(blk[0:2].copy().view(np.float16)[0])
            dmin = dtype(blk[2:4].copy().view(np.float16)[0])
            sc, qs = blk[4:16], blk[16:144]
            for j in range(4):
                s0, m0 = q4k_scale_min(sc, 2 * j)
                s1, m1 = q4k_scale_min(sc, 2 * j + 1)
                q = qs[32 * j:32 * j + 32]
                out[i, 64 * j:64 * j + 32] = dtype(d * dtype(s0)) * (q & 15) - dtype(dmin * dtype(m0))
                out[i, 64 * j + 32:64 * j + 64] = dtype(d * dtype(s1)) * (q >> 4) - dtype(dmin * dtype(m1))
        else:
            ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
            sc = blk[192:208].view(np.int8).astype(np.int64)
            d = dtype(blk[208:210].copy().view(np.float16)[0])
            vals = np.empty(256, dtype=np.int64)
            for half in range(2):
                l = np.arange(32)
                a, c, h = ql[64 * half + l], ql[64 * half + 32 + l], qh[32 * half + l]
                vals[128 * half + l] = (a & 15) | ((h & 3) << 4)
                vals[128 * half + 32 + l] = (c & 15) | (((h >> 2) & 3) << 4)
                vals[128 * half + 64 + l] = (a >> 4) | (((h >> 4) & 3) << 4)
                vals[128 * half + 96 + l] = (c >> 4) | (((h >> 6) & 3) << 4)
            scale = np.repeat(sc, 16).astype(dtype)
            out[i] = dtype(d) * scale * (vals - 32).astype(dtype)
    return out.ravel()


def dequant(qtype, w):
    """fp32, in the reference's DequantizeRow operation order."""
    return _dequant(qtype, w, np.float32)


def dequant_f64(qtype, w):
    return _dequant(qtype, w, np.float64)
