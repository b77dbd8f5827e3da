"""Pin the CPU oracle's matvec, elementwise, attention and model restatements.

Each function is checked against the reference's own tests where they exist
(tests/golden/reference_kats.json) and against an independent float64 numpy
computation with an error bound proportional to the f32 accumulation error
(sum |w_i x_i| * n * 2^-24), which fails for a dropped term, a wrong index or
a transposed operand.
"""
import json
import os

import numpy as np
import pytest

from helpers import (F32, Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0, Q8_K, QUANT_TYPES, GEOM, NAMES,
                     q4_0_block, random_matrix)

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def f64_matvec_bound(wdec, x):
    """float64 W x and the f32 sequential-accumulation error bound."""
    w64, x64 = wdec.astype(np.float64), np.asarray(x, np.float64)
    y = w64 @ x64
    mag = np.abs(w64) @ np.abs(x64)
    return y, mag * (wdec.shape[1] + 2) * 2.0 ** -24


# -------------------------------------------------------------- matvec

@pytest.mark.parametrize("t", QUANT_TYPES)
def test_quant_matvec_matches_float64_of_decoded_rows(orc, t):
    rng = np.random.default_rng(1000 + t)
    qk, _ = GEOM[t]
    in_dim, out_dim = 2 * max(qk, 64) if qk == 32 else 512, 37
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    wdec = orc.dequantize_rows(t, raw, in_dim, out_dim)
    ref, bound = f64_matvec_bound(wdec, x)
    for y in (orc.matvec_quant(t, raw, out_dim, in_dim, x),
              orc.quantized_matvec_reference(t, raw, in_dim, out_dim, x),
              orc.dispatch_matvec(t, raw, in_dim, out_dim, x, threads=4)):
        assert np.all(np.abs(y - ref) <= bound), NAMES[t]


def test_quantized_reference_is_decode_then_sequential_dot(orc):
    """compute.rs:185-229 accumulates the decoded row in input order, so it is
    bit-identical to a float32 sequential loop over the decoded row."""
    rng = np.random.default_rng(7)
    for t in QUANT_TYPES:
        qk, _ = GEOM[t]
        in_dim = 256 if qk == 256 else 64
        raw = random_matrix(t, 3, in_dim, rng)
        x = rng.normal(0, 1, in_dim).astype(np.float32)
        wdec = orc.dequantize_rows(t, raw, in_dim, 3)
        y = orc.quantized_matvec_reference(t, raw, in_dim, 3, x)
        for r in range(3):
            acc = np.float32(0)
            for i in range(in_dim):
                acc = np.float32(acc + np.float32(wdec[r, i] * x[i]))
            assert y[r] == acc
        if t not in (Q4_0, Q6_K):  # decode-then-dot kernels share the order exactly
            assert np.array_equal(orc.matvec_quant(t, raw, 3, in_dim, x), y)


def _diag_q4_0_row(blocks):
    scales = [0x3C00, 0x3800, 0x3A00, 0x4000, 0xBC00, 0x3400, 0x3E00, 0xB800]
    row = b""
    for bi in range(blocks):
        qs = [(((j * 5 + bi * 3 + 1) & 0xF) | (((j * 7 + bi * 11 + 9) & 0xF) << 4)) for j in range(16)]
        row += q4_0_block(scales[bi % 8], qs)
    return row


def _diag_input(pattern, n):
    if pattern == "constant":
        return np.full(n, 1.25, np.float32)
    if pattern == "ramp":
        return (np.arange(n, dtype=np.float32) * np.float32(0.125) - np.float32(2.0)).astype(np.float32)
    if pattern == "alternating":
        return np.where(np.arange(n) % 2 == 0, 1.5, -0.75).astype(np.float32)
    state, out = 0x12345678, []
    for _ in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out.append(np.float32(np.float32(state >> 8) / np.float32(16777215.0)) * np.float32(2) - np.float32(1))
    return np.array(out, np.float32)


@pytest.mark.parametrize("blocks", [4, 48])
@pytest.mark.parametrize("pattern", ["constant", "ramp", "alternating", "pseudo_random"])
def test_q4_0_fused_vs_materialized_reference_test(orc, blocks, pattern):
    """quant.rs:1940-2044 with its tolerance 1e-5 + 1e-6*scale."""
    n = blocks * 32
    row = _diag_q4_0_row(blocks)
    x = _diag_input(pattern, n)
    ref = orc.quantized_matvec_reference(Q4_0, row, n, 1, x)[0]
    fused = orc.matvec_quant(Q4_0, row, 1, n, x)[0]
    scale = max(abs(ref), abs(fused), 1.0)
    assert abs(fused - ref) <= 1e-5 + 1e-6 * scale


def test_row_range_local_indexing(orc):
    """quant.rs:2177-2209."""
    raw = b"".join(q4_0_block(0x3C00, [(0x88 + r) & 0xFF] * 16) for r in range(3))
    full = orc.matvec_quant(Q4_0, raw, 3, 32, np.ones(32))
    local = orc.matvec_quant_row_range(Q4_0, raw, 3, 32, np.ones(32), 1, 2, 1)
    assert local[0] == full[2]
    with pytest.raises(orc.OracleError, match="exceeds out_dim|row range"):
        orc.matvec_quant_row_range(Q4_0, raw, 3, 32, np.ones(32), 1, 3, 1)
    raw6 = bytearray(3 * 210)
    for r in range(3):
        raw6[r * 210 + 208:r * 210 + 210] = (0x3C00).to_bytes(2, "little")
    full = orc.matvec_quant(Q6_K, bytes(raw6), 3, 256, np.ones(256))
    local = orc.matvec_quant_row_range(Q6_K, bytes(raw6), 3, 256, np.ones(256), 1, 2, 1)
    assert local[0] == full[2]


def test_q4_0_parallel_dispatch_qwen_shape(orc):
    """streaming_model.rs:3331-3411: 1536x1536 Q4_0 with the reference's LCG
    payload (f16 scales rounded to nearest even), 4 threads vs the scalar
    reference, max_abs < 1e-2."""
    in_dim = out_dim = 1536
    bpr = in_dim // 32
    raw = np.zeros((out_dim, bpr, 18), np.uint8)
    seed = 0xC0FFEE
    m = 0xFFFFFFFF
    for r in range(out_dim):
        s = seed
        seed = (seed * 1664525 + 1013904223) & m
        for b in range(bpr):
            s = (s * 1664525 + 1013904223) & m
            d = np.float32(0.05) + (np.float32(s >> 8) / np.float32(1 << 24)) * np.float32(0.45)
            raw[r, b, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
            for k in range(16):
                s = (s * 1664525 + 1013904223) & m
                raw[r, b, 2 + k] = (s & 0xF) | (((s >> 4) & 0xF) << 4)
    x = np.sin(np.arange(in_dim, dtype=np.float32) * np.float32(0.0137) - np.float32(0.5)).astype(np.float32)
    x = (x * np.float32(0.7)).astype(np.float32)
    ref = orc.quantized_matvec_reference(Q4_0, raw.reshape(-1), in_dim, out_dim, x)
    y = orc.dispatch_matvec(Q4_0, raw.reshape(-1), in_dim, out_dim, x, threads=4)
    assert np.max(np.abs(y - ref)) < 1e-2
    assert np.array_equal(y, orc.dispatch_matvec(Q4_0, raw.reshape(-1), in_dim, out_dim, x, threads=1))


def test_q6_k_partition_boundaries(orc):
    """streaming_model.rs:3413-3457: 129 rows split over 4 threads equal the
    scalar path exactly."""
    raw = np.zeros((129, 210), np.uint8)
    for r in range(129):
        raw[r, :128] = (np.arange(128) + r) & 0xFF
        raw[r, 128:192] = (np.arange(64) * 3) & 0xFF
        raw[r, 192:208] = 1
        raw[r, 208:210] = [0x00, 0x3C]
    x = np.cos(np.arange(256, dtype=np.float32) * np.float32(0.011)).astype(np.float32)
    y1 = orc.dispatch_matvec(Q6_K, raw.reshape(-1), 256, 129, x, threads=1)
    y4 = orc.dispatch_matvec(Q6_K, raw.reshape(-1), 256, 129, x, threads=4)
    assert np.array_equal(y1, y4)


def test_every_format_fused_vs_reference(orc):
    """compute.rs:698-767: a 0x11-filled block per format, tolerance
    1e-2 + 1e-5*scale."""
    cases = {Q4_0: (32, {0: 0x3C00}), Q8_0: (32, {0: 0x3C00}), Q2_K: (256, {80: 0x3C00, 82: 0}),
             Q3_K: (256, {108: 0x3C00}), Q4_K: (256, {0: 0x3C00, 2: 0}), Q5_K: (256, {0: 0x3C00, 2: 0}),
             Q6_K: (256, {208: 0x3C00})}
    for t, (n, fields) in cases.items():
        blk = bytearray([0x11] * GEOM[t][1])
        for off, v in fields.items():
            blk[off:off + 2] = v.to_bytes(2, "little")
        raw = bytes(blk) * 2
        x = np.cos(np.arange(n, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
        ref = orc.quantized_matvec_reference(t, raw, n, 2, x)
        opt = orc.matvec_quant(t, raw, 2, n, x)
        assert np.all(np.abs(ref - opt) <= 1e-2 + 1e-5 * np.maximum(np.abs(ref), np.abs(opt)))
    blk = bytearray([0x11] * 292)
    blk[0:4] = np.float32(1.0).tobytes()
    raw = bytes(blk) * 2
    x = np.cos(np.arange(256, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    assert np.allclose(orc.quantized_matvec_reference(Q8_K, raw, 256, 2, x), orc.matvec_quant(Q8_K, raw, 2, 256, x))


def test_matvec_validation_messages(orc):
    with pytest.raises(orc.OracleError, match="not divisible"):
        orc.matvec_quant(Q8_0, bytes(34), 1, 31, np.ones(31))
    with pytest.raises(orc.OracleError, match="weight truncated"):
        orc.matvec_quant(Q8_0, bytes(33), 1, 32, np.ones(32))


# ---------------------------------------------------------- F32 / backend

def test_f32_kats(orc):
    c = KATS["compute"]
    k = c["f32_matvec"]
    assert orc.matvec_f32_reference(k["w"], k["input"], k["output"], k["x"]).tolist() == k["expect"]
    k = c["f32_row_range"]
    assert orc.matvec_f32_reference_row_range(k["w"], k["input"], k["output"], k["x"], k["row_start"],
                                              k["row_count"]).tolist() == k["expect"]
    b = KATS["backend"]
    for key in ("matvec_2x2", "matvec_3x2"):
        k = b[key]
        for simd in (False, True):
            for th in (1, 2):
                y = orc.backend_matvec_f32(k["w"], k["shape_in_out"][0], k["shape_in_out"][1], k["x"], th, simd)
                assert y.tolist() == k["expect"]
    with pytest.raises(orc.OracleError, match="arity mismatch"):
        orc.backend_matvec_f32([1, 2, 3, 4, 5, 6], 3, 2, [1, 1], 1, False)


def test_f32_avx2_order_is_eight_fma_lanes(orc):
    """simd.rs:21-45: lane l accumulates fma(a[i], b[i], acc) for i = l mod 8,
    lanes summed in order, then a mul-then-add remainder.  Checked against a
    numpy emulation (np.float32 math with an exact fma from float64) and a
    float64 bound."""
    rng = np.random.default_rng(3)
    for n in (8, 13, 64, 4099):
        a = rng.normal(0, 1, n).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32)
        acc = np.zeros(8, np.float32)
        m = n // 8 * 8
        for i in range(0, m, 8):
            acc = (a[i:i + 8].astype(np.float64) * b[i:i + 8] + acc).astype(np.float32)  # fma: one rounding
        tot = np.float32(-0.0)
        for l in range(8):
            tot = np.float32(tot + acc[l])
        for i in range(m, n):
            tot = np.float32(tot + np.float32(a[i] * b[i]))
        y = orc.backend_matvec_f32(a, n, 1, b, 1, True)
        assert y[0] == tot
        ref, bound = f64_matvec_bound(a.reshape(1, -1), b)
        assert abs(y[0] - ref[0]) <= bound[0]


# ------------------------------------------------------------ elementwise

def test_elementwise_kats(orc):
    c = KATS["compute"]
    k = c["rmsnorm"]
    assert np.allclose(orc.rms_norm(k["x"], k["w"], k["eps"]), k["expect"], atol=k["tol"], rtol=0)
    k = c["swiglu"]
    out = orc.swiglu(k["gate"], k["up"])
    assert abs(out[0] - (-1.0 / (1.0 + np.exp(1.0)) * 2.0)) < 1e-6 and out[1] == 0.0
    assert abs(out[2] - (2.0 / (1.0 + np.exp(-2.0)) * 4.0)) < 1e-6
    b = KATS["backend"]
    assert orc.silu(b["silu"]["x"])[0] == 0.0 and abs(orc.silu(b["silu"]["x"])[1] - 0.7310586) < 1e-4
    assert abs(orc.softmax(b["softmax"]["x"])[0] - 1 / 3) < 1e-4
    assert np.all(np.abs(orc.rms_norm([1, 1, 1, 1], [1, 1, 1, 1], 1e-5) - 1.0) < 1e-3)


def test_elementwise_against_float64(orc):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, 4096).astype(np.float32)
    w = rng.normal(1, 0.1, 4096).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
    assert np.max(np.abs(orc.rms_norm(x, w, 1e-5) - ref) / np.abs(ref).max()) < 1e-5
    assert np.allclose(orc.silu(x), x64 / (1 + np.exp(-x64)), rtol=1e-6, atol=1e-6)
    s = orc.softmax(x)
    e = np.exp(x64 - x64.max())
    assert np.allclose(s, e / e.sum(), rtol=1e-5, atol=1e-9) and abs(s.sum() - 1) < 1e-5


# ------------------------------------------------------------------ RoPE

def test_rope_kats_and_float64(orc):
    c = KATS["compute"]
    k = c["rope_identity"]
    q, kk = orc.rope(k["q"], k["q"], k["pos"], k["head_dim"], 1, 1, k["theta"])
    assert q.tolist() == k["q"] and kk.tolist() == k["q"]
    k = c["rope_pos1"]
    q, kk = orc.rope(k["q"], k["q"], k["pos"], k["head_dim"], 1, 1, k["theta"])
    assert abs(q[0] - np.cos(1.0)) < 1e-6 and abs(q[1] - np.sin(1.0)) < 1e-6 and np.array_equal(q, kk)
    rng = np.random.default_rng(9)
    hd, qh, kvh = 128, 4, 2
    qv = rng.normal(0, 1, qh * hd).astype(np.float32)
    kv = rng.normal(0, 1, kvh * hd).astype(np.float32)
    for pos in (1, 17, 511):
        qo, ko = orc.rope(qv, kv, pos, hd, qh, kvh, 10000.0)
        half = hd // 2
        inv = 10000.0 ** (-2.0 * np.arange(half) / hd)
        ang = inv * pos
        for src, dst, nh in ((qv, qo, qh), (kv, ko, kvh)):
            s = src.reshape(nh, hd).astype(np.float64)
            a, b = s[:, :half], s[:, half:]
            exp = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], 1)
            assert np.max(np.abs(dst.reshape(nh, hd) - exp)) < 1e-6 * (1 + pos)
            assert np.allclose(np.linalg.norm(dst.reshape(nh, hd), axis=1), np.linalg.norm(s, axis=1), rtol=1e-5)


# ------------------------------------------------------------- attention

def np_attention(q, kh, vh, kc, vc, hist, qh, kvh, hd):
    k = np.concatenate([kh.reshape(hist, kvh, hd), kc.reshape(1, kvh, hd)]).astype(np.float64)
    v = np.concatenate([vh.reshape(hist, kvh, hd), vc.reshape(1, kvh, hd)]).astype(np.float64)
    out = np.zeros((qh, hd))
    for h in range(qh):
        g = h * kvh // qh
        s = k[:, g, :] @ q.reshape(qh, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, g, :]
    return out.reshape(-1)


def test_attention_kat_and_float64(orc):
    k = KATS["compute"]["gqa"]
    out = orc.attention(k["q"], [], [], k["k_cur"], k["v_cur"], k["hist"], k["qh"], k["kvh"], k["hd"])
    assert out.tolist() == k["expect"]
    rng = np.random.default_rng(11)
    for hist, qh, kvh, hd in ((0, 4, 2, 8), (5, 4, 4, 16), (300, 32, 8, 128), (1023, 8, 1, 64)):
        q = rng.normal(0, 1, qh * hd).astype(np.float32)
        kh = rng.normal(0, 1, hist * kvh * hd).astype(np.float32)
        vh = rng.normal(0, 1, hist * kvh * hd).astype(np.float32)
        kc = rng.normal(0, 1, kvh * hd).astype(np.float32)
        vc = rng.normal(0, 1, kvh * hd).astype(np.float32)
        got = orc.attention(q, kh, vh, kc, vc, hist, qh, kvh, hd)
        ref = np_attention(q, kh, vh, kc, vc, hist, qh, kvh, hd)
        assert np.max(np.abs(got - ref)) < 1e-5 * (1 + np.abs(ref).max())
    # closed form: identical keys -> uniform weights -> mean of V
    kh = np.tile(kc, 9)
    vh = rng.normal(0, 1, 9 * kvh * hd).astype(np.float32)
    got = orc.attention(q, kh, vh, kc, vc, 9, qh, kvh, hd)
    mean_v = np.concatenate([vh.reshape(9, kvh, hd), vc.reshape(1, kvh, hd)]).mean(0)
    assert np.allclose(got.reshape(qh, hd), mean_v[np.arange(qh) * kvh // qh], atol=1e-5)


def test_attention_parity_threads_bit_identical(orc):
    """The parity-run accelerator spreads attention heads over threads; each
    head's arithmetic is unchanged, so the output is bit-identical to the
    single-threaded restatement (which the timed CPU baseline runs)."""
    rng = np.random.default_rng(12)
    hist, qh, kvh, hd = 700, 32, 8, 128
    args = [rng.normal(0, 1, n).astype(np.float32) for n in (qh * hd, hist * kvh * hd, hist * kvh * hd, kvh * hd,
                                                              kvh * hd)]
    one = orc.attention(*args, hist, qh, kvh, hd)
    orc.set_parity_threads(8)
    try:
        many = orc.attention(*args, hist, qh, kvh, hd)
    finally:
        orc.set_parity_threads(0)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))


def test_argmax_tie_and_nan_rules(orc):
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax([float("nan"), 5.0, 6.0]) == 0
    assert orc.argmax([1.0, float("nan"), 6.0, 6.0]) == 2
    assert orc.argmax([float("-inf")] * 4) == 0
    assert orc.argmax([]) == 0


# ------------------------------------------------------------ synthetic

def test_synth_generator_splitmix64(orc):
    """SplitMix64 (Steele/Lea/Flood 2014): seed 0 first output 0xE220A8397B1DCDAF."""
    assert orc.synth_u64(0, 0) == 0xE220A8397B1DCDAF

    def sm(seed, i):
        z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    for seed, i in ((1, 0), (12345, 77), (2 ** 63, 10 ** 9)):
        assert orc.synth_u64(seed, i) == sm(seed, i)
    # Q8_0 synthetic blocks: codes in [-127, 127], |d| scale near sigma/127
    raw = orc.synth_blocks(Q8_0, 42, 0, 4096, 0.02 / 127).reshape(4096, 34)
    q = raw[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127 and abs(q.astype(float).mean()) < 1
    d = raw[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    assert 0.6 * 0.02 / 127 < d.mean() < 1.0 * 0.02 / 127  # E|N(0,s)| = 0.798 s
    # contiguous ranges compose: blocks [10, 20) equal the tail of [0, 20)
    for t in QUANT_TYPES + [F32]:
        a = orc.synth_blocks(t, 7, 0, 20, 0.02)
        b = orc.synth_blocks(t, 7, 10, 10, 0.02)
        bs = GEOM[t][1]
        assert np.array_equal(a[10 * bs:], b), NAMES[t]


# ------------------------------------------------------------------ model

def _tiny_model(rng, cfg, qtype=Q8_0, bias=False):
    d, f, V = cfg["embedding_length"], cfg["feed_forward_length"], cfg["vocab_size"]
    qd = cfg["head_count"] * cfg["head_dim"]
    kvd = cfg["head_count_kv"] * cfg["head_dim"]
    T = {}

    sigma = {F32: 1.0, Q8_0: 0.5}.get(qtype, 0.004)

    def mat(name, ne0, ne1, t=qtype):
        T[name] = (t, ne0, ne1, random_matrix(t, ne1, ne0, rng, sigma))

    mat("token_embd.weight", d, V)
    mat("output.weight", d, V)
    T["output_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
    for i in range(cfg["block_count"]):
        T[f"blk.{i}.attn_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
        T[f"blk.{i}.ffn_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
        mat(f"blk.{i}.attn_q.weight", d, qd)
        mat(f"blk.{i}.attn_k.weight", d, kvd)
        mat(f"blk.{i}.attn_v.weight", d, kvd)
        mat(f"blk.{i}.attn_output.weight", qd, d)
        mat(f"blk.{i}.ffn_gate.weight", d, f)
        mat(f"blk.{i}.ffn_up.weight", d, f)
        mat(f"blk.{i}.ffn_down.weight", f, d)
        if bias:
            for n, w in (("attn_q", qd), ("attn_k", kvd), ("attn_v", kvd)):
                T[f"blk.{i}.{n}.bias"] = (F32, w, 1, rng.normal(0, 0.5, w).astype(np.float32))
    return T


class NumpyLlama:
    """Independent float64 forward (vectorised, written from the op order in
    model_executor.rs:9-23 and streaming_model.rs:909-1305)."""

    def __init__(self, orc, cfg, T):
        self.cfg = cfg
        self.W = {}
        for n, (t, ne0, ne1, arr) in T.items():
            w = arr.view(np.float32) if t == F32 else orc.dequantize_rows(t, arr, ne0, ne1)
            self.W[n] = np.asarray(w, np.float64).reshape(ne1, ne0) if ne1 > 1 else np.asarray(w, np.float64).reshape(-1)
        self.k, self.v = [], []

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.cfg["rms_eps"]) * w

    def rope(self, v, pos, nh):
        hd = self.cfg["head_dim"]
        half = hd // 2
        ang = (np.float32(self.cfg["rope_freq_base"]) ** (-2.0 * np.arange(half) / hd)) * pos
        s = v.reshape(nh, hd)
        a, b = s[:, :half], s[:, half:]
        return np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], 1).reshape(-1)

    def forward(self, tok, pos):
        c, W = self.cfg, self.W
        qh, kvh, hd = c["head_count"], c["head_count_kv"], c["head_dim"]
        x = W["token_embd.weight"][tok].copy()
        new_k, new_v = [], []
        for i in range(c["block_count"]):
            p = f"blk.{i}."
            h = self.rms(x, W[p + "attn_norm.weight"])
            q, k, v = W[p + "attn_q.weight"] @ h, W[p + "attn_k.weight"] @ h, W[p + "attn_v.weight"] @ h
            if p + "attn_q.bias" in W:
                q, k, v = q + W[p + "attn_q.bias"], k + W[p + "attn_k.bias"], v + W[p + "attn_v.bias"]
            q, k = self.rope(q, pos, qh), self.rope(k, pos, kvh)
            K = np.stack([*(self.k[t][i] for t in range(pos)), k]).reshape(pos + 1, kvh, hd)
            V = np.stack([*(self.v[t][i] for t in range(pos)), v]).reshape(pos + 1, kvh, hd)
            att = np.zeros((qh, hd))
            for hh in range(qh):
                g = hh * kvh // qh
                s = K[:, g] @ q.reshape(qh, hd)[hh] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                att[hh] = (pr / pr.sum()) @ V[:, g]
            x = x + W[p + "attn_output.weight"] @ att.reshape(-1)
            h = self.rms(x, W[p + "ffn_norm.weight"])
            g_, u = W[p + "ffn_gate.weight"] @ h, W[p + "ffn_up.weight"] @ h
            x = x + W[p + "ffn_down.weight"] @ (g_ / (1 + np.exp(-g_)) * u)
            new_k.append(k)
            new_v.append(v)
        self.k.append(new_k)
        self.v.append(new_v)
        return self.rms(x, W["output_norm.weight"])

    def logits(self, hidden):
        return self.W["output.weight"] @ hidden


TINY = dict(vocab_size=64, context_length=32, embedding_length=64, block_count=2, feed_forward_length=96,
            head_count=4, head_count_kv=2, head_dim=16, rms_eps=1e-5, rope_freq_base=10000.0)


@pytest.mark.parametrize("qtype,bias", [(Q8_0, False), (Q4_K, False), (F32, True)])
def test_model_forward_matches_float64_numpy(orc, qtype, bias):
    cfg = dict(TINY)
    if qtype == Q4_K:
        cfg.update(embedding_length=256, feed_forward_length=256, head_dim=64)
    rng = np.random.default_rng(21)
    T = _tiny_model(rng, cfg, qtype, bias)
    m = orc.Model(cfg, T, kv_capacity=16, threads=2)
    ref = NumpyLlama(orc, cfg, T)
    for pos, tok in enumerate([3, 17, 60, 1, 9]):
        h = m.forward(tok, pos)
        h64 = ref.forward(tok, pos)
        assert np.max(np.abs(h - h64)) < 2e-4 * max(1.0, np.abs(h64).max()), pos
        lg = m.logits(h)
        lg64 = ref.logits(h64)
        assert np.max(np.abs(lg - lg64)) < 2e-4 * max(1.0, np.abs(lg64).max())
    m.close()


def test_model_generate_is_deterministic_and_follows_stop_rules(orc):
    rng = np.random.default_rng(22)
    T = _tiny_model(rng, TINY)
    a = orc.Model(TINY, T, kv_capacity=32)
    b = orc.Model(TINY, T, kv_capacity=32)
    ta, _ = a.generate([1, 2, 3], 10)
    tb, _ = b.generate([1, 2, 3], 10)
    assert ta == tb and len(ta) == 10
    # the terminal forward is skipped: 3 prompt + 9 decode forwards
    assert a.seq_len == 12
    a.reset()
    t2, _ = a.generate([1, 2, 3], 10, eos=ta[4])
    assert t2 == ta[:ta.index(ta[4])]
    a.close()
    b.close()
