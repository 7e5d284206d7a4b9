"""Known-answer blocks for the GGUF types the reference pins only by its written layout
(docs/research/2026-10-03-gguf-on-metal.md:18-36).  Each test builds blocks whose decoded values are
fixed by construction from a rule stated in that text (a field value, an index rule, a bit), so a
transposed index, a wrong shift or a dropped term in the oracle fails here.  IQ4_NL / IQ4_XS are
not described in the reference; their tests check the layout against the published ggml format
only (parity unpinned)."""
import numpy as np
import pytest

import oracle as O

IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float32)


def f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def f16v(v):
    return np.float32(np.float16(v))


def test_q4_1_value_is_d_nib_plus_m():
    """Q4_1: f16 d, f16 m, qs[16]; value = d * nib + m, low nibbles are values 0..15."""
    blk = np.zeros(20, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16b(2.0), f16b(0.5)
    blk[4:] = np.arange(16, dtype=np.uint8) | ((15 - np.arange(16, dtype=np.uint8)) << 4)
    got = O.gguf_dequantize(blk[None], "Q4_1")
    want = np.concatenate([2.0 * np.arange(16) + 0.5, 2.0 * (15 - np.arange(16)) + 0.5]).astype(np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bit", [0, 5, 15, 16, 20, 31])
def test_q5_0_fifth_bit_is_bit_j_of_qh(bit):
    """Q5_0: f16 d, u32 qh, qs[16]; value j = d * ((nib | bit j of qh << 4) - 16)."""
    blk = np.zeros(22, dtype=np.uint8)
    blk[0:2] = f16b(1.0)
    blk[2:6] = np.array([1 << bit], dtype=np.uint32).view(np.uint8)
    got = O.gguf_dequantize(blk[None], "Q5_0")
    want = np.full(32, -16.0, dtype=np.float32)
    want[bit] = 0.0
    assert np.array_equal(got, want)


def test_q5_1_value_is_d_q_plus_m():
    """Q5_1: f16 d, f16 m, u32 qh, qs[16]; value = d * q + m with q = nib | bit j of qh << 4."""
    blk = np.zeros(24, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16b(0.25), f16b(-3.0)
    blk[4:8] = np.array([0x80000001], dtype=np.uint32).view(np.uint8)   # values 0 and 31
    blk[8 + 15] = 0xF0                                                 # value 31: nib 15
    blk[8 + 0] = 0x07                                                  # value 0: nib 7
    got = O.gguf_dequantize(blk[None], "Q5_1")
    want = np.full(32, -3.0, dtype=np.float32)
    want[0] = 0.25 * (7 + 16) - 3.0
    want[31] = 0.25 * (15 + 16) - 3.0
    assert np.array_equal(got, want)


def test_q2_k_scale_and_min_per_16_values():
    """Q2_K: scales[16], qs[64], f16 d, f16 dmin; value = (d * (sc & 15)) * q - dmin * (sc >> 4) per 16
    values.  With every q = 3 the index layout of q drops out and each 16-value group shows its byte."""
    blk = np.zeros(84, dtype=np.uint8)
    sc = (np.arange(16, dtype=np.uint8) & 15) | (((15 - np.arange(16)) & 15).astype(np.uint8) << 4)
    blk[0:16] = sc
    blk[16:80] = 0xFF
    blk[80:82], blk[82:84] = f16b(0.5), f16b(0.125)
    got = O.gguf_dequantize(blk[None], "Q2_K").reshape(16, 16)
    for g in range(16):
        want = np.float32(np.float32(0.5) * np.float32(sc[g] & 15)) * 3 - np.float32(0.125) * np.float32(sc[g] >> 4)
        assert np.all(got[g] == want), g


def q3k_block(s6, qs_byte, hmask_byte, d=1.0):
    """Q3_K: hmask[32], qs[64], scales[12], f16 d.  Signed 6-bit scales: 4 low bits in bytes 0..7
    (low nibbles first), 2 high bits in bytes 8..11 (2 bits per sub-block group of four), minus 32."""
    blk = np.zeros(110, dtype=np.uint8)
    blk[0:32] = hmask_byte
    blk[32:96] = qs_byte
    u = (np.asarray(s6) + 32).astype(np.uint8)
    sc = np.zeros(12, dtype=np.uint8)
    for i in range(16):
        sc[i % 8] |= (u[i] & 15) << (4 * (i // 8))
        sc[8 + i % 4] |= ((u[i] >> 4) & 3) << (2 * (i // 4))
    blk[96:108] = sc
    blk[108:110] = f16b(d)
    return blk


def test_q3_k_scales_and_inverted_high_mask():
    s6 = np.array([-32, -31, -7, -1, 0, 1, 2, 5, 9, 13, 17, 21, 25, 29, 30, 31])
    # every q2 = 3: with the high bit set, value = d * s6 * 3; with it clear, d * s6 * (3 - 4)
    got_hi = O.gguf_dequantize(q3k_block(s6, 0xFF, 0xFF, 0.5)[None], "Q3_K").reshape(16, 16)
    got_lo = O.gguf_dequantize(q3k_block(s6, 0xFF, 0x00, 0.5)[None], "Q3_K").reshape(16, 16)
    for g in range(16):
        assert np.all(got_hi[g] == np.float32(0.5 * s6[g]) * 3), g
        assert np.all(got_lo[g] == np.float32(0.5 * s6[g]) * -1), g


def k_scales(sc, mn):
    """Twelve bytes for eight 6-bit (scale, min) pairs: sub-blocks 0..3 take the low 6 bits of bytes
    0..3 (scales) and 4..7 (mins); 4..7 take a nibble of bytes 8..11 plus the top 2 bits of bytes
    0..3 (scales) or 4..7 (mins)."""
    b = np.zeros(12, dtype=np.uint8)
    for s in range(8):
        if s < 4:
            b[s] |= sc[s] & 63
            b[4 + s] |= mn[s] & 63
        else:
            j = s - 4
            b[8 + j] |= (sc[s] & 15) | ((mn[s] & 15) << 4)
            b[j] |= (sc[s] >> 4) << 6
            b[4 + j] |= (mn[s] >> 4) << 6
    return b


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K"])
def test_k45_scale_packing_chunks_and_fifth_bit(name):
    """Q4_K / Q5_K: (d * sc) * q - dmin * m per 32 values.  The 128 nibble bytes are four 32-byte
    chunks; chunk c holds sub-block 2c in its low nibbles and 2c + 1 in its high nibbles.  Q5_K: bit s
    of qh[j % 32] is the fifth bit of value j in sub-block s."""
    rng = np.random.default_rng(3)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 32 if name == "Q5_K" else 16, 256)
    ts = 144 if name == "Q4_K" else 176
    blk = np.zeros(ts, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16b(0.0625), f16b(0.03125)
    blk[4:16] = k_scales(sc, mn)
    qs_off = 16 if name == "Q4_K" else 48
    for v in range(256):
        s, i = v // 32, v % 32
        blk[qs_off + 32 * (s // 2) + i] |= (q[v] & 15) << (4 * (s % 2))
        if name == "Q5_K":
            blk[16 + i] |= ((q[v] >> 4) & 1) << s
    got = O.gguf_dequantize(blk[None], name)
    d, dmin = np.float32(0.0625), np.float32(0.03125)
    want = np.array([np.float32(d * np.float32(sc[v // 32])) * np.float32(q[v]) - np.float32(dmin * np.float32(mn[v // 32]))
                     for v in range(256)], dtype=np.float32)
    assert np.array_equal(got, want)


def test_q6_k_half_index_rule():
    """Q6_K: ql[128], qh[64], i8 scales[16], f16 d; (d * sc) * (q - 32) per 16 values.  Value r of half
    h reads ql[64h + r % 64] >> 4 * (r / 64) and qh[32h + r % 32] >> 2 * (r / 32)."""
    rng = np.random.default_rng(4)
    q = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16)
    blk = np.zeros(210, dtype=np.uint8)
    for v in range(256):
        h, r = v // 128, v % 128
        blk[64 * h + r % 64] |= (q[v] & 15) << (4 * (r // 64))
        blk[128 + 32 * h + r % 32] |= ((q[v] >> 4) & 3) << (2 * (r // 32))
    blk[192:208] = sc.astype(np.int8).view(np.uint8)
    blk[208:210] = f16b(0.125)
    got = O.gguf_dequantize(blk[None], "Q6_K")
    want = np.array([np.float32(np.float32(0.125) * np.float32(sc[v // 16])) * np.float32(q[v] - 32) for v in range(256)],
                    dtype=np.float32)
    assert np.array_equal(got, want)


def test_iq4_nl_layout():
    """IQ4_NL (ggml format; parity unpinned): f16 d, qs[16]; value j = d * T[nib], low nibbles first."""
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = f16b(0.5)
    blk[2:] = np.arange(16, dtype=np.uint8) | ((15 - np.arange(16, dtype=np.uint8)) << 4)
    got = O.gguf_dequantize(blk[None], "IQ4_NL")
    assert np.array_equal(got, np.float32(0.5) * np.concatenate([IQ4NL, IQ4NL[::-1]]))


def test_iq4_xs_layout():
    """IQ4_XS (ggml format; parity unpinned): f16 d, u16 scales_h, u8 scales_l[4], qs[128];
    ls = (scales_l nibble) | (2 bits of scales_h) << 4; value = d * (ls - 32) * T[nib]."""
    ls = np.array([0, 1, 31, 32, 33, 40, 62, 63])
    sl = np.zeros(4, dtype=np.uint8)
    sh = 0
    for ib in range(8):
        sl[ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
        sh |= int((ls[ib] >> 4) & 3) << (2 * ib)
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = f16b(0.25)
    blk[2:4] = np.array([sh], dtype=np.uint16).view(np.uint8)
    blk[4:8] = sl
    nib = np.arange(16, dtype=np.uint8)
    for ib in range(8):
        blk[8 + 16 * ib: 24 + 16 * ib] = nib | ((15 - nib) << 4)
    got = O.gguf_dequantize(blk[None], "IQ4_XS").reshape(8, 32)
    for ib in range(8):
        a = np.float32(np.float32(0.25) * np.float32(ls[ib] - 32))
        assert np.array_equal(got[ib], a * np.concatenate([IQ4NL, IQ4NL[::-1]])), ib
