"""Pin the CPU oracle's block decoders (oracle/ramforge_oracle.c).

Checks, in order of strength:
  * the reference's own known-answer tests (tests/golden/reference_kats.json,
    copied from core/src/quant.rs tests);
  * an exhaustive f16 check against IEEE binary16 (numpy), with the
    reference's subnormal rule stated as a closed form;
  * inverse bit-mapping tests: each input bit/field is set on its own and the
    test asserts WHICH output elements change and by how much, with the element
    index written from the GGUF/ggml layout specification (input -> output,
    the opposite direction of the decoders).  The two places where the
    reference deviates from ggml (Q5_K high-bit byte, Q3_K scale index) are
    asserted explicitly.
"""
import json
import os

import numpy as np
import pytest

from helpers import (Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0, Q8_K, GEOM, h16, q4_0_block, q5_0_block,
                     q8_0_block)

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


# ------------------------------------------------------------------- f16

def test_f16_known_answers(orc):
    for bits, val in KATS["f16"]["cases"]:
        assert orc.f16_to_f32(bits) == val


def test_f16_exhaustive_against_ieee_with_reference_subnormal_rule(orc):
    """Normal/inf/NaN halves decode to IEEE binary16 values (NaN payload kept:
    float32 bits = sign | 0xFF<<23 | frac<<13).  Subnormal halves decode to
    frac * 2^-25, i.e. half the IEEE value: quant.rs:46-55 counts one shift
    too many while normalising."""
    bits = np.arange(65536, dtype=np.uint32)
    # decode through the F16 row path so float bits never pass through a
    # Python float (which would quiet signalling NaNs)
    got = orc.dequantize_row(1, bits.astype(np.uint16).view(np.uint8), 65536)
    ieee = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    exp = (bits >> 10) & 0x1F
    frac = bits & 0x3FF
    sign = np.where(bits & 0x8000, -1.0, 1.0)
    normal = (exp > 0) & (exp < 31)
    assert np.array_equal(got[normal], ieee[normal])
    sub = exp == 0
    expect_sub = (sign[sub] * frac[sub].astype(np.float64) * 2.0 ** -25).astype(np.float32)
    assert np.array_equal(got[sub].view(np.uint32), expect_sub.view(np.uint32))
    special = exp == 31
    expect_bits = ((bits[special] & 0x8000) << 16) | (0xFF << 23) | (frac[special] << 13)
    assert np.array_equal(got[special].view(np.uint32), expect_bits.astype(np.uint32))
    # the quirk is material: a subnormal scale halves a whole block
    assert orc.f16_to_f32(0x0001) == 2.0 ** -25 and float(np.uint16(1).view(np.float16)) == 2.0 ** -24


# ------------------------------------------------------- reference KATs

def test_q5_0_high_bits_kat(orc):
    k = KATS["q5_0_high_bits"]
    out = orc.dequantize_row(Q5_0, q5_0_block(k["d"], k["qh"], k["qs"]), 32)
    for i, v in k["expect_idx"].items():
        assert out[int(i)] == v


def test_q5_0_ggml_vector_kat(orc):
    k = KATS["q5_0_ggml_vector"]
    out = orc.dequantize_row(Q5_0, q5_0_block(k["d"], k["qh"], k["qs"]), 32)
    assert out.tolist() == k["expect"]


def test_q5_0_row_decode_and_matvec_kat(orc):
    k = KATS["q5_0_row_matvec"]
    raw = b"".join(q5_0_block(d, qh, [0] * 16) for d, qh in k["rows"])
    dec = orc.dequantize_row(Q5_0, raw, 64)
    for i, v in k["expect_decoded"].items():
        assert dec[int(i)] == v
    y = orc.matvec_quant(Q5_0, raw, 2, 32, np.ones(32, np.float32))
    assert y.tolist() == k["expect_y"]


def test_q4_0_kats(orc):
    for d, byte, val in KATS["q4_0_decode"]["cases"]:
        assert np.all(orc.dequantize_row(Q4_0, q4_0_block(d, [byte] * 16), 32) == val)
    k = KATS["q4_0_edge_nibbles"]
    out = orc.dequantize_row(Q4_0, q4_0_block(k["d"], k["qs"]), 32, np.full(32, 123.0, np.float32))
    for i, v in k["expect_idx"].items():
        assert out[int(i)] == v
    assert (out < 0).any() and (out > 0).any()
    k = KATS["q4_0_multi_block"]
    for row, expect in ((k["row0"], k["row0_expect"]), (k["row1"], k["row1_expect"])):
        raw = b"".join(q4_0_block(d, [b] * 16) for d, b in row)
        out = orc.dequantize_row(Q4_0, raw, 64)
        for lo, hi, v in expect:
            assert np.all(out[lo:hi] == v)


def test_q4_0_validation_keeps_destination(orc):
    """quant.rs:1718-1730: errors carry the reference wording and leave the
    destination untouched."""
    dst = np.full(32, 17.0, np.float32)
    with pytest.raises(orc.OracleError, match="row truncated"):
        orc.dequantize_row(Q4_0, bytes(17), 32, dst)
    assert np.all(dst == 17.0)
    dst = np.full(31, 29.0, np.float32)
    with pytest.raises(orc.OracleError, match="not divisible"):
        orc.dequantize_row(Q4_0, q4_0_block(0x3C00, [0x88] * 16), 31, dst)
    assert np.all(dst == 29.0)


def test_q8_0_kats(orc):
    k = KATS["q8_0_decode_ones"]
    assert np.all(orc.dequantize_row(Q8_0, q8_0_block(k["d"], [k["q"]] * 32), 32) == k["expect"])
    k = KATS["q8_0_direct"]
    out = orc.dequantize_row(Q8_0, q8_0_block(k["d"], k["q"]), 32, np.full(32, 777.0, np.float32))
    for i, v in k["expect_idx"].items():
        assert out[int(i)] == v
    assert np.all(out == np.array(k["q"], np.float32) * 0.5)
    for row in KATS["q8_0_multi_row"]["rows"]:
        raw = b"".join(q8_0_block(d, [q] * 32) for d, q in row)
        out = orc.dequantize_row(Q8_0, raw, 64)
        for bi, (d, q) in enumerate(row):
            assert np.all(out[32 * bi:32 * bi + 32] == np.float32(q) * np.float32(orc.f16_to_f32(d)))
    with pytest.raises(orc.OracleError, match="row truncated"):
        orc.dequantize_row(Q8_0, bytes(33), 32)


def _k_ones_block(t):
    if t == Q4_K:
        return h16(0x3C00) + h16(0) + bytes([1] * 12) + bytes([0x11] * 128)
    if t == Q5_K:
        return h16(0x3C00) + h16(0) + bytes([1] * 12) + bytes(32) + bytes([0x11] * 128)
    if t == Q8_K:
        return np.float32(1.0).tobytes() + bytes([1] * 256) + bytes(32)
    raise ValueError(t)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q8_K])
def test_k_quant_all_ones_kat(orc, t):
    assert np.all(orc.dequantize_row(t, _k_ones_block(t), 256) == KATS["k_quant_ones"]["expect"])


def test_matvec_kats(orc):
    m = KATS["matvec"]
    row = q4_0_block(0x3C00, [0x99] * 16)
    assert abs(orc.matvec_quant(Q4_0, row * 2, 2, 32, np.ones(32))[0] - m["q4_0"]) < 1e-3
    row = q8_0_block(0x3C00, [1] * 32)
    assert abs(orc.matvec_quant(Q8_0, row * 2, 2, 32, np.full(32, 2.0))[0] - m["q8_0"]) < 1e-3
    for t, key in ((Q4_K, "q4_k"), (Q5_K, "q5_k"), (Q8_K, "q8_k")):
        y = orc.matvec_quant(t, _k_ones_block(t) * 2, 2, 256, np.ones(256))
        assert abs(y[0] - m[key]) < 1e-3


# ---------------------------------------------------- inverse bit mapping

def _decode(orc, t, blk):
    return orc.dequantize_row(t, bytes(blk), GEOM[t][0]).astype(np.float64)


def test_q6_k_bit_mapping(orc):
    """ggml Q6_K: ql byte 64h+c -> low nibble elem 128h+c, high nibble elem
    128h+64+c; qh byte 32h+l bit pair k -> elem 128h+32k+l; scale byte 8h+j ->
    elems 128h+32(j//2)+16(j%2)+[0,16); value (d*sc)*(q-32)."""
    base = bytearray(210)
    base[192:208] = bytes([1] * 16)
    base[208:210] = h16(0x3C00)
    ref = _decode(orc, Q6_K, base)
    assert np.all(ref == -32.0)
    for b in range(128):
        h, c = divmod(b, 64)
        for nib, shift in ((0, 0), (1, 4)):
            blk = bytearray(base)
            blk[b] = 5 << shift
            got = _decode(orc, Q6_K, blk)
            e = 128 * h + c + 64 * nib
            diff = np.nonzero(got != ref)[0]
            assert diff.tolist() == [e] and got[e] == 5 - 32
    for b in range(64):
        h, l = divmod(b, 32)
        for k in range(4):
            blk = bytearray(base)
            blk[128 + b] = 2 << (2 * k)
            got = _decode(orc, Q6_K, blk)
            e = 128 * h + 32 * k + l
            assert np.nonzero(got != ref)[0].tolist() == [e] and got[e] == 32 - 32
    for j in range(16):
        h, jj = divmod(j, 8)
        blk = bytearray(base)
        blk[192 + j] = 0xFD  # -3
        got = _decode(orc, Q6_K, blk)
        lo = 128 * h + 32 * (jj // 2) + 16 * (jj % 2)
        assert np.nonzero(got != ref)[0].tolist() == list(range(lo, lo + 16))
        assert np.all(got[lo:lo + 16] == 96.0)


def test_q2_k_bit_mapping(orc):
    """ggml Q2_K: qs byte 32n+c bit pair k -> elem 128n+32k+c; scale byte
    8n+2k+h -> elems 128n+32k+16h+[0,16); value (d*(sc&15))*q - dmin*(sc>>4)."""
    base = bytearray(84)
    base[0:16] = bytes([0x01] * 16)  # sc=1, m=0
    base[80:82] = h16(0x3C00)
    base[82:84] = h16(0x3800)  # dmin 0.5
    ref = _decode(orc, Q2_K, base)
    assert np.all(ref == 0.0)
    for b in range(64):
        n, c = divmod(b, 32)
        for k in range(4):
            blk = bytearray(base)
            blk[16 + b] = 3 << (2 * k)
            got = _decode(orc, Q2_K, blk)
            e = 128 * n + 32 * k + c
            assert np.nonzero(got != ref)[0].tolist() == [e] and got[e] == 3.0
    for s in range(16):
        n, r = divmod(s, 8)
        k, h = divmod(r, 2)
        blk = bytearray(base)
        blk[s] = 0x42  # sc=2, m=4
        got = _decode(orc, Q2_K, blk)
        lo = 128 * n + 32 * k + 16 * h
        assert np.nonzero(got != ref)[0].tolist() == list(range(lo, lo + 16))
        assert np.all(got[lo:lo + 16] == -2.0)  # 2*0 - 0.5*4


def test_q3_k_bit_mapping_and_reference_scale_index(orc):
    """Q3_K: qs byte 32n+c bit pair j -> elem 128n+32j+c; hmask byte l bit
    4n+j -> elem 128n+32j+l (+4 when set).  Scales: the reference uses the
    6-bit scales 0..7 for BOTH 128-element halves (quant.rs:551-561), so
    scale i<4 drives elems 32i+[0,16) and 128+32i+[0,16); scale i>=4 drives
    32(i-4)+16+[0,16) in both halves; scales 8..15 (which ggml would use for
    the second half) drive nothing."""
    base = bytearray(110)
    # every 6-bit scale = 33 (value 1): low nibble 1 in bytes 0..7, bit pattern 10b in bits of bytes 8..11
    for i in range(8):
        base[96 + i] = 0x11
    for i in range(4):
        base[104 + i] = 0xAA  # high 2 bits = 2 for every scale: 0x21 = 33
    base[108:110] = h16(0x3C00)
    ref = _decode(orc, Q3_K, base)
    assert np.all(ref == -4.0)  # q = 0 - 4, scale 33-32 = 1
    for b in range(64):
        n, c = divmod(b, 32)
        for j in range(4):
            blk = bytearray(base)
            blk[32 + b] = 3 << (2 * j)
            got = _decode(orc, Q3_K, blk)
            e = 128 * n + 32 * j + c
            assert np.nonzero(got != ref)[0].tolist() == [e] and got[e] == -1.0
    for l in range(32):
        for bit in range(8):
            n, j = divmod(bit, 4)
            blk = bytearray(base)
            blk[l] = 1 << bit
            got = _decode(orc, Q3_K, blk)
            e = 128 * n + 32 * j + l
            assert np.nonzero(got != ref)[0].tolist() == [e] and got[e] == 0.0

    def set_scale(blk, i, v):
        # inverse of the kmask unpack: low nibble / high 2 bits locations per scale index
        lo_byte, lo_shift = (i % 8, 4 * (i // 8))
        hi_byte, hi_shift = (8 + i % 4, 2 * (i // 4))
        blk[96 + lo_byte] = (blk[96 + lo_byte] & ~(0xF << lo_shift)) | ((v & 0xF) << lo_shift)
        blk[96 + hi_byte] = (blk[96 + hi_byte] & ~(0x3 << hi_shift)) | ((v >> 4) << hi_shift)

    for i in range(16):
        blk = bytearray(base)
        set_scale(blk, i, 35)  # value 3
        got = _decode(orc, Q3_K, blk)
        changed = np.nonzero(got != ref)[0].tolist()
        if i < 4:
            expect = list(range(32 * i, 32 * i + 16)) + list(range(128 + 32 * i, 128 + 32 * i + 16))
        elif i < 8:
            j = i - 4
            expect = list(range(32 * j + 16, 32 * j + 32)) + list(range(128 + 32 * j + 16, 128 + 32 * j + 32))
        else:
            expect = []
        assert changed == expect, f"scale {i}"
        assert np.all(got[expect] == -12.0)


def _k4_scale_bytes(j, sc, m):
    s = bytearray(12)
    for i in range(8):  # every other sub-block: sc=1, m=0
        if i < 4:
            s[i] |= 1
        else:
            s[i + 4] |= 1
    if j < 4:
        s[j] = (s[j] & ~63) | sc
        s[j + 4] = (s[j + 4] & ~63) | m
    else:
        s[j + 4] = (sc & 0xF) | ((m & 0xF) << 4)
        s[j - 4] = (s[j - 4] & 63) | ((sc >> 4) << 6)
        s[j] = (s[j] & 63) | ((m >> 4) << 6)
    return bytes(s)


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_q4_k_q5_k_scale_packing_and_nibble_mapping(orc, t):
    """get_scale_min 6-bit packing: sub-block j uses (sc, m); value (d*sc)*q -
    dmin*m; qs byte 32g+c low nibble -> elem 64g+c, high -> 64g+32+c."""
    qs_off = 16 if t == Q4_K else 48
    for j in range(8):
        for sc, m in ((37, 5), (63, 63), (2, 49)):
            blk = bytearray(GEOM[t][1])
            blk[0:2] = h16(0x3C00)
            blk[2:4] = h16(0x3800)
            blk[4:16] = _k4_scale_bytes(j, sc, m)
            got = _decode(orc, t, blk)
            for s in range(8):
                val = -0.5 * m if s == j else 0.0
                assert np.all(got[32 * s:32 * s + 32] == val), (j, s)
            for b in range(128):
                g, c = divmod(b, 32)
                for nib in (0, 1):
                    bb = bytearray(blk)
                    bb[qs_off + b] = 7 << (4 * nib)
                    e = 64 * g + 32 * nib + c
                    got2 = _decode(orc, t, bb)
                    assert np.nonzero(got2 != got)[0].tolist() == [e]
                    s = e // 32
                    scv = sc if s == j else 1
                    mv = m if s == j else 0
                    assert got2[e] == np.float32(np.float32(scv) * 7) - np.float32(0.5 * mv)
                if j > 0:
                    break


def test_q5_k_reference_high_bit_byte(orc):
    """quant.rs:319/329: the high bit of element l in group g comes from
    qh[8g + l/8] bit 2g (low half) / 2g+1 (high half), so one qh bit covers
    8 consecutive elements (ggml uses qh[l], one element per bit)."""
    base = bytearray(176)
    base[0:2] = h16(0x3C00)
    base[4:16] = _k4_scale_bytes(0, 1, 0)
    ref = _decode(orc, Q5_K, base)
    assert np.all(ref == 0.0)
    for B in range(32):
        g, t = divmod(B, 8)
        for bit in range(8):
            blk = bytearray(base)
            blk[16 + B] = 1 << bit
            changed = np.nonzero(_decode(orc, Q5_K, blk) != ref)[0].tolist()
            if t < 4 and bit in (2 * g, 2 * g + 1):
                lo = 64 * g + 32 * (bit - 2 * g) + 8 * t
                assert changed == list(range(lo, lo + 8)), (B, bit)
            else:
                assert changed == [], (B, bit)


def test_q8_k_and_q8_0_sign(orc):
    blk = np.float32(0.25).tobytes() + bytes((np.arange(256) - 128).astype(np.int8).view(np.uint8)) + bytes(32)
    assert np.array_equal(orc.dequantize_row(Q8_K, blk, 256), (np.arange(256) - 128).astype(np.float32) * 0.25)
    blk = q8_0_block(0x4000, list(range(-16, 16)))
    assert np.array_equal(orc.dequantize_row(Q8_0, blk, 32), np.arange(-16, 16, dtype=np.float32) * 2.0)


def test_zero_code_patch_decodes_to_zero(orc):
    """The GPU tests' zero-code patch (tests/helpers.py) against the oracle's
    decode: patched elements are exact zeros in every row and block."""
    from helpers import GEOM, NAMES, Q3_K, Q4_0, Q5_0, Q6_K, Q8_0, Q8_K, random_matrix, zero_code_patch

    rng = np.random.default_rng(1)
    for t in (Q8_0, Q4_0, Q5_0, Q8_K, Q6_K, Q3_K):
        qk, _ = GEOM[t]
        elems = [5, 21] if qk == 32 else list(range(5, 256, 16))
        raw = zero_code_patch(t, random_matrix(t, 4, 2 * qk, rng), elems)
        deq = orc.dequantize_rows(t, raw, 2 * qk, 4)
        for blk in range(2):
            assert (deq[:, [blk * qk + e for e in elems]] == 0).all(), NAMES[t]


def test_synthetic_k_quant_weights_are_zero_mean(orc):
    """The generator draws K-quant mins at the mean code times the scale, so
    d*sc*q - dmin*m has mean near zero (a biased random model repeats one
    token forever)."""
    for t, mul in ((12, 0.02 / (63 * 15)), (13, 0.02 / (63 * 31)), (10, 0.02 / (15 * 3))):
        raw = orc.synth_blocks(t, 77, 0, 4096, mul)
        w = orc.dequantize_rows(t, raw, 256, 4096).astype(np.float64)
        assert abs(w.mean()) < 0.05 * w.std(), (t, w.mean(), w.std())
