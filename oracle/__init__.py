"""CPU oracle: ctypes wrapper of liboracle.so (oracle/ramforge_oracle.c).

TEST INFRASTRUCTURE ONLY.  This package is the parity checker and the timed
CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it; the product (ramforge_amd/) never does.

Each function restates one reference function of RAMforge's legacy CPU decode
path with the same f32 operation order; the C source cites the reference
file:line for every function.  Pinning: tests/test_oracle_*.py check it
against the reference's own known-answer tests (tests/golden/), closed forms
and independent float64 computations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ROW_COUNT_ALL = 0xFFFFFFFFFFFFFFFF


class OracleError(RuntimeError):
    pass


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile."""
    if force and os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)
    subprocess.run(["make", "-C", HERE, "-s"], check=True)
    return LIB_PATH


class Tensor(C.Structure):
    _fields_ = [("type", C.c_uint32), ("data", C.c_void_p), ("nbytes", C.c_size_t),
                ("ne0", C.c_size_t), ("ne1", C.c_size_t)]


class Layer(C.Structure):
    _fields_ = [(n, Tensor) for n in (
        "attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up",
        "ffn_down", "attn_q_bias", "attn_k_bias", "attn_v_bias")]


class Config(C.Structure):
    _fields_ = [("vocab_size", C.c_size_t), ("context_length", C.c_size_t), ("embedding_length", C.c_size_t),
                ("block_count", C.c_size_t), ("feed_forward_length", C.c_size_t), ("head_count", C.c_size_t),
                ("head_count_kv", C.c_size_t), ("head_dim", C.c_size_t), ("rms_eps", C.c_float),
                ("rope_freq_base", C.c_float)]


_sz, _vp, _fp, _u32, _u64 = C.c_size_t, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint64
_SIGS = {
    "orc_last_error": (C.c_char_p, []),
    "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_block_geometry": (C.c_int, [_u32, C.POINTER(_sz), C.POINTER(_sz)]),
    "orc_dequantize_row": (C.c_int, [_u32, _vp, _sz, _sz, _fp, _sz]),
    "orc_matvec_quant": (C.c_int, [_u32, _vp, _sz, _sz, _sz, _fp, _sz, _fp, _sz]),
    "orc_matvec_quant_row_range": (C.c_int, [_u32, _vp, _sz, _sz, _sz, _fp, _sz, _fp, _sz, _sz, _sz]),
    "orc_quantized_matvec_reference": (C.c_int, [_u32, _vp, _sz, _sz, _sz, _fp, _sz, _fp, _sz]),
    "orc_matvec_f32_reference": (C.c_int, [_fp, _sz, _sz, _sz, _fp, _sz, _fp, _sz]),
    "orc_matvec_f32_reference_row_range": (C.c_int, [_fp, _sz, _sz, _sz, _fp, _sz, _fp, _sz, _sz, _sz]),
    "orc_backend_matvec_f32": (C.c_int, [_fp, _sz, _sz, _sz, _fp, _sz, _fp, _sz, C.c_int, C.c_int]),
    "orc_dispatch_matvec": (C.c_int, [_u32, _vp, _sz, _sz, _sz, _fp, _sz, _fp, _sz, C.c_int, C.c_int]),
    "orc_rms_norm": (C.c_int, [_fp, _fp, _sz, C.c_float, _fp]),
    "orc_add": (C.c_int, [_fp, _fp, _sz, _fp]),
    "orc_mul": (C.c_int, [_fp, _fp, _sz, _fp]),
    "orc_silu": (C.c_int, [_fp, _sz, _fp]),
    "orc_swiglu": (C.c_int, [_fp, _fp, _sz, _fp]),
    "orc_softmax": (C.c_int, [_fp, _sz]),
    "orc_rope": (C.c_int, [_fp, _sz, _fp, _sz, _sz, _sz, _sz, _sz, C.c_float]),
    "orc_attention": (C.c_int, [_fp, _sz, _fp, _fp, _sz, _fp, _fp, _sz, _sz, _sz, _sz, _sz, _fp, _sz]),
    "orc_argmax": (_u32, [_fp, _sz]),
    "orc_model_create": (C.c_int, [C.POINTER(Config), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor),
                                   C.POINTER(Layer), _sz, C.c_int, C.c_int, C.POINTER(_vp)]),
    "orc_model_destroy": (None, [_vp]),
    "orc_model_reset": (C.c_int, [_vp]),
    "orc_model_seq_len": (_sz, [_vp]),
    "orc_model_forward": (C.c_int, [_vp, _u32, _sz, _fp]),
    "orc_model_logits": (C.c_int, [_vp, _fp, _fp]),
    "orc_model_generate": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int64, _vp, C.POINTER(_sz), _fp]),
    "orc_synth_u64": (_u64, [_u64, _u64]),
    "orc_set_parity_threads": (None, [C.c_int]),
    "orc_synth_blocks": (C.c_int, [_u32, _u64, _u64, _u64, C.c_double, _vp]),
}

_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _LIB = L
    return _LIB


def _err() -> str:
    return lib().orc_last_error().decode()


def _chk(rc: int) -> None:
    if rc:
        raise OracleError(_err())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), dtype=np.uint8) if isinstance(a, (bytes, bytearray))
                                else np.asarray(a, dtype=np.uint8))


def geometry(t: int):
    qk, bs = C.c_size_t(), C.c_size_t()
    _chk(lib().orc_block_geometry(t, C.byref(qk), C.byref(bs)))
    return qk.value, bs.value


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def dequantize_row(t: int, raw, n: int, out=None) -> np.ndarray:
    b = _u8(raw)
    o = np.zeros(n, np.float32) if out is None else out
    _chk(lib().orc_dequantize_row(t, b.ctypes.data, b.nbytes, n, o.ctypes.data, o.size))
    return o


def dequantize_rows(t: int, raw, in_dim: int, rows: int) -> np.ndarray:
    qk, bs = geometry(t)
    rb = in_dim // qk * bs
    b = _u8(raw)
    out = np.zeros((rows, in_dim), np.float32)
    for r in range(rows):
        seg = b[r * rb:(r + 1) * rb]
        _chk(lib().orc_dequantize_row(t, seg.ctypes.data, seg.nbytes, in_dim, out[r].ctypes.data, in_dim))
    return out


def matvec_quant(t: int, raw, out_dim: int, in_dim: int, x) -> np.ndarray:
    b, xv = _u8(raw), _f32(x)
    y = np.zeros(out_dim, np.float32)
    _chk(lib().orc_matvec_quant(t, b.ctypes.data, b.nbytes, out_dim, in_dim, xv.ctypes.data, xv.size,
                                y.ctypes.data, y.size))
    return y


def matvec_quant_row_range(t: int, raw, out_dim: int, in_dim: int, x, y_len: int, row_start: int,
                           row_count=None) -> np.ndarray:
    b, xv = _u8(raw), _f32(x)
    y = np.full(y_len, -999.0, np.float32)
    _chk(lib().orc_matvec_quant_row_range(t, b.ctypes.data, b.nbytes, out_dim, in_dim, xv.ctypes.data, xv.size,
                                          y.ctypes.data, y.size, row_start,
                                          ROW_COUNT_ALL if row_count is None else row_count))
    return y


def quantized_matvec_reference(t: int, raw, input_dim: int, output_dim: int, x) -> np.ndarray:
    b, xv = _u8(raw), _f32(x)
    y = np.zeros(output_dim, np.float32)
    _chk(lib().orc_quantized_matvec_reference(t, b.ctypes.data, b.nbytes, input_dim, output_dim, xv.ctypes.data,
                                              xv.size, y.ctypes.data, y.size))
    return y


def matvec_f32_reference(w, input_dim: int, output_dim: int, x) -> np.ndarray:
    wv, xv = _f32(w), _f32(x)
    y = np.zeros(output_dim, np.float32)
    _chk(lib().orc_matvec_f32_reference(wv.ctypes.data, wv.size, input_dim, output_dim, xv.ctypes.data, xv.size,
                                        y.ctypes.data, y.size))
    return y


def matvec_f32_reference_row_range(w, input_dim, output_dim, x, row_start, row_count) -> np.ndarray:
    wv, xv = _f32(w), _f32(x)
    y = np.zeros(row_count, np.float32)
    _chk(lib().orc_matvec_f32_reference_row_range(wv.ctypes.data, wv.size, input_dim, output_dim, xv.ctypes.data,
                                                  xv.size, y.ctypes.data, y.size, row_start, row_count))
    return y


def backend_matvec_f32(w, in_dim: int, out_dim: int, x, threads: int = 1, use_simd: bool = True) -> np.ndarray:
    wv, xv = _f32(w), _f32(x)
    y = np.zeros(out_dim, np.float32)
    _chk(lib().orc_backend_matvec_f32(wv.ctypes.data, wv.size, in_dim, out_dim, xv.ctypes.data, xv.size,
                                      y.ctypes.data, y.size, threads, int(use_simd)))
    return y


def dispatch_matvec(t: int, data, in_dim: int, out_dim: int, x, threads: int = 1, use_simd: bool = True):
    d = _f32(data) if t == 0 else _u8(data)
    xv = _f32(x)
    y = np.zeros(out_dim, np.float32)
    _chk(lib().orc_dispatch_matvec(t, d.ctypes.data, d.nbytes, in_dim, out_dim, xv.ctypes.data, xv.size,
                                   y.ctypes.data, y.size, threads, int(use_simd)))
    return y


def rms_norm(x, w, eps: float) -> np.ndarray:
    xv, wv = _f32(x), _f32(w)
    o = np.zeros_like(xv)
    _chk(lib().orc_rms_norm(xv.ctypes.data, wv.ctypes.data, xv.size, eps, o.ctypes.data))
    return o


def silu(x) -> np.ndarray:
    xv = _f32(x)
    o = np.zeros_like(xv)
    _chk(lib().orc_silu(xv.ctypes.data, xv.size, o.ctypes.data))
    return o


def swiglu(g, u) -> np.ndarray:
    gv, uv = _f32(g), _f32(u)
    o = np.zeros_like(gv)
    _chk(lib().orc_swiglu(gv.ctypes.data, uv.ctypes.data, gv.size, o.ctypes.data))
    return o


def add(a, b) -> np.ndarray:
    av, bv = _f32(a), _f32(b)
    o = np.zeros_like(av)
    _chk(lib().orc_add(av.ctypes.data, bv.ctypes.data, av.size, o.ctypes.data))
    return o


def mul(a, b) -> np.ndarray:
    av, bv = _f32(a), _f32(b)
    o = np.zeros_like(av)
    _chk(lib().orc_mul(av.ctypes.data, bv.ctypes.data, av.size, o.ctypes.data))
    return o


def softmax(v) -> np.ndarray:
    o = _f32(v).copy()
    _chk(lib().orc_softmax(o.ctypes.data, o.size))
    return o


def rope(q, k, pos: int, head_dim: int, qh: int, kvh: int, theta: float):
    qv, kv = _f32(q).copy(), _f32(k).copy()
    _chk(lib().orc_rope(qv.ctypes.data, qv.size, kv.ctypes.data, kv.size, pos, head_dim, qh, kvh, theta))
    return qv, kv


def attention(q, k_hist, v_hist, k_cur, v_cur, hist_len: int, qh: int, kvh: int, hd: int) -> np.ndarray:
    qv, kh, vh, kc, vc = (_f32(a) for a in (q, k_hist, v_hist, k_cur, v_cur))
    o = np.zeros(qh * hd, np.float32)
    _chk(lib().orc_attention(qv.ctypes.data, qv.size, kh.ctypes.data, vh.ctypes.data, kh.size, kc.ctypes.data,
                             vc.ctypes.data, kc.size, hist_len, qh, kvh, hd, o.ctypes.data, o.size))
    return o


def argmax(logits) -> int:
    v = _f32(logits)
    return int(lib().orc_argmax(v.ctypes.data, v.size))


def set_parity_threads(n: int) -> None:
    """Row-parallel matvec for every format in parity runs (identical
    results); 0 restores the reference's threading policy."""
    lib().orc_set_parity_threads(n)


def model_tensors(specs) -> dict:
    """Host payloads of ramforge_amd.synthetic specs, byte-identical to the
    device generator: name -> (ggml_type, ne0, ne1, array)."""
    out = {}
    for s in specs:
        if s.ggml_type == 0 and s.constant == s.constant:  # not NaN: constant fill
            arr = np.full(s.ne0 * s.ne1, s.constant, np.float32)
        else:
            qk, _ = geometry(s.ggml_type)
            nb = s.ne0 // qk * s.ne1
            arr = synth_blocks(s.ggml_type, s.seed, 0, nb, s.scale_mul)
            if s.ggml_type == 0:
                arr = arr.view(np.float32)
        out[s.name] = (s.ggml_type, s.ne0, s.ne1, arr)
    return out


def synth_u64(seed: int, index: int) -> int:
    return int(lib().orc_synth_u64(seed, index))


def synth_blocks(t: int, seed: int, first_block: int, n_blocks: int, scale_mul: float) -> np.ndarray:
    _, bs = geometry(t)
    out = np.zeros(n_blocks * bs, np.uint8)
    _chk(lib().orc_synth_blocks(t, seed, first_block, n_blocks, scale_mul, out.ctypes.data))
    return out


class Model:
    """Dense llama decode on the CPU (oracle restatement of the reference)."""

    LAYER_FIELDS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate",
                    "ffn_up", "ffn_down")

    def __init__(self, cfg: dict, tensors: dict, kv_capacity: int, threads: int = 1, use_simd: bool = True):
        """``tensors`` maps GGUF names to (ggml_type, ne0, ne1, numpy payload)."""
        self.cfg = cfg
        self._keep = []
        c = Config(**{k: cfg[k] for k, _ in Config._fields_})

        def mk(name):
            if name not in tensors:
                return Tensor()
            t, ne0, ne1, arr = tensors[name]
            a = np.ascontiguousarray(arr)
            self._keep.append(a)
            return Tensor(t, a.ctypes.data, a.nbytes, ne0, ne1)

        layers = (Layer * cfg["block_count"])()
        for i in range(cfg["block_count"]):
            for f in self.LAYER_FIELDS:
                setattr(layers[i], f, mk(f"blk.{i}.{f}.weight"))
            for f in ("attn_q", "attn_k", "attn_v"):
                setattr(layers[i], f + "_bias", mk(f"blk.{i}.{f}.bias"))
        te, on = mk("token_embd.weight"), mk("output_norm.weight")
        out = mk("output.weight")
        h = C.c_void_p()
        _chk(lib().orc_model_create(C.byref(c), C.byref(te), C.byref(on), C.byref(out) if out.data else None,
                                    layers, kv_capacity, threads, int(use_simd), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        _chk(lib().orc_model_reset(self.h))

    @property
    def seq_len(self) -> int:
        return int(lib().orc_model_seq_len(self.h))

    def forward(self, token: int, pos: int) -> np.ndarray:
        o = np.zeros(self.cfg["embedding_length"], np.float32)
        _chk(lib().orc_model_forward(self.h, token, pos, o.ctypes.data))
        return o

    def logits(self, final_hidden) -> np.ndarray:
        fh = _f32(final_hidden)
        o = np.zeros(self.cfg["vocab_size"], np.float32)
        _chk(lib().orc_model_logits(self.h, fh.ctypes.data, o.ctypes.data))
        return o

    def generate(self, prompt, max_tokens: int, eos: int = -1):
        p = np.ascontiguousarray(np.asarray(prompt, np.uint32))
        out = np.zeros(max(max_tokens, 1), np.uint32)
        margin = np.zeros(max(max_tokens, 1), np.float32)
        n = C.c_size_t()
        _chk(lib().orc_model_generate(self.h, p.ctypes.data, p.size, max_tokens, eos, out.ctypes.data,
                                      C.byref(n), margin.ctypes.data))
        return [int(t) for t in out[:n.value]], margin[:max_tokens]
