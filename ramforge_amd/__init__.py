"""ramforge_amd — MI355X (gfx950) decode-step tier for RAMforge.

Python host mirror of RAMforge's compute interface for the decode hot path,
over the C ABI of ``libramforge_hip.so`` (include/ramforge_hip.h).  Reference
paths are relative to crates/ramforge-{core,runtime}/src of RAMforge.

* :class:`Context`     — compute backend handle + device-memory ledger
                          (CpuBackend::new, backend.rs:72-84; MemoryBudget,
                          memory.rs:30-384, on the device domain)
* :func:`matvec`       — quant::matvec_<fmt>[_row_range] (quant.rs:898-1489)
* :class:`GpuBackend`  — ComputeBackend (backend.rs:27-52) for device buffers
* :func:`matvec_backend` — compute_dispatch::matvec_backend (compute_dispatch.rs:40-58)
* :func:`attention_checked` — ops::attention_checked (ops.rs:49-69)
* :class:`GpuLlamaModel` — forward_single_streaming / compute_logits /
                          generate_impl (streaming_model.rs:909-1370,
                          inference.rs:445-759) on VRAM-resident weights.

All compute runs in the HIP library; this module only moves host arrays and
passes device pointers.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import RF_ALL_ROWS, RF_ERR_BUDGET, RF_ERR_INVALID, RF_ERR_IO, ModelConfig, RamforgeError

__all__ = [
    "GGML", "BLOCK_GEOMETRY", "Context", "DeviceArray", "RamforgeError", "ModelConfig",
    "matvec", "dequantize_rows", "attention_checked", "apply_rope", "rmsnorm", "add", "mul",
    "silu", "swiglu", "softmax", "argmax", "GpuBackend", "GpuTensor", "matvec_backend",
    "GpuLlamaModel", "row_bytes",
]


class GGML:
    """ggml type ids (core/src/types.rs:238-292)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q5_0 = 6
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    BF16 = 30

    NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K",
             12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 30: "BF16"}


# (elements per block, bytes per block): core/src/quant.rs:24-37
BLOCK_GEOMETRY = {
    GGML.F32: (1, 4), GGML.F16: (1, 2), GGML.BF16: (1, 2),
    GGML.Q4_0: (32, 18), GGML.Q5_0: (32, 22), GGML.Q8_0: (32, 34),
    GGML.Q2_K: (256, 84), GGML.Q3_K: (256, 110), GGML.Q4_K: (256, 144),
    GGML.Q5_K: (256, 176), GGML.Q6_K: (256, 210), GGML.Q8_K: (256, 292),
}


def row_bytes(ggml_type: int, in_dim: int) -> int:
    qk, bs = BLOCK_GEOMETRY[ggml_type]
    if in_dim % qk:
        raise ValueError(f"{GGML.NAMES[ggml_type]} in_dim {in_dim} not divisible by {qk}")
    return in_dim // qk * bs


def _ptr(a) -> Optional[int]:
    if a is None:
        return None
    if isinstance(a, DeviceArray):
        return a.ptr
    if isinstance(a, int):
        return a
    raise TypeError(f"expected a DeviceArray or device address, got {type(a).__name__}")


class DeviceArray:
    """A ledger-charged device buffer with a numpy view of its shape/dtype."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, shape, dtype, charge: str):
        self.ctx = ctx
        self.ptr = ptr
        self.nbytes = nbytes
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.charge = charge

    def upload(self, host: np.ndarray) -> "DeviceArray":
        h = np.ascontiguousarray(host)
        if h.nbytes > self.nbytes:
            raise ValueError(f"upload of {h.nbytes} bytes into a {self.nbytes}-byte buffer")
        _lib.check(self.ctx.lib.rf_upload(self.ctx.handle, self.ptr, h.ctypes.data, h.nbytes))
        return self

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes > self.nbytes:
            raise ValueError(f"view of {out.nbytes} bytes over a {self.nbytes}-byte buffer")
        _lib.check(self.ctx.lib.rf_download(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            _lib.check(self.ctx.lib.rf_vram_release(self.ctx.handle, self.charge.encode()))
            self.ptr = 0


class CapturedGraph:
    """A hipGraph recorded from the compute stream (rf_capture_begin/end)."""

    def __init__(self, ctx: "Context", handle: int):
        self.ctx = ctx
        self.handle = handle

    def replay(self, reps: int = 1) -> float:
        """Launch the graph `reps` times; returns the mean ms per replay."""
        ms = C.c_float(0.0)
        _lib.check(self.ctx.lib.rf_graph_replay(self.ctx.handle, self.handle, reps, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        if self.handle:
            _lib.check(self.ctx.lib.rf_graph_destroy(self.ctx.handle, self.handle))
            self.handle = None


class _Capture:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        self.graph: Optional[CapturedGraph] = None

    def __enter__(self) -> "_Capture":
        _lib.check(self.ctx.lib.rf_capture_begin(self.ctx.handle))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = C.c_void_p()
        rc = self.ctx.lib.rf_capture_end(self.ctx.handle, C.byref(h))
        if exc_type is None:
            _lib.check(rc)
            self.graph = CapturedGraph(self.ctx, h.value)
        elif rc == _lib.RF_OK and h.value:  # the body raised: drop the graph it made
            self.ctx.lib.rf_graph_destroy(self.ctx.handle, h.value)
        return False


class Context:
    """Device context: compute + copy streams and the VRAM ledger."""

    _serial = 0

    def __init__(self, device: int = 0, vram_budget_bytes: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        _lib.check(self.lib.rf_ctx_create(device, vram_budget_bytes, C.byref(h)))
        self.handle = h

    # lifecycle
    def close(self) -> None:
        if self.handle:
            self.lib.rf_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self) -> None:
        _lib.check(self.lib.rf_ctx_synchronize(self.handle))

    def reserve(self, attention_bytes: int = 0, matmul_bytes: int = 0, staging_bytes: int = 0,
                fixed: bool = True) -> None:
        """rf_ctx_reserve: size the context workspaces now; with ``fixed`` no
        later call grows them (a call that needs more raises instead)."""
        _lib.check(self.lib.rf_ctx_reserve(self.handle, attention_bytes, matmul_bytes, staging_bytes, int(fixed)))

    def attention_workspace_bytes(self, max_positions: int, n_heads: int, n_kv_heads: int, head_dim: int) -> int:
        return int(self.lib.rf_attention_workspace_bytes(max_positions, n_heads, n_kv_heads, head_dim))

    def matmul_workspace_bytes(self, out_dim: int, in_dim: int, n_tokens: int) -> int:
        return int(self.lib.rf_matmul_workspace_bytes(out_dim, in_dim, n_tokens))

    @property
    def compute_stream(self) -> int:
        return self.lib.rf_ctx_compute_stream(self.handle)

    @property
    def copy_stream(self) -> int:
        return self.lib.rf_ctx_copy_stream(self.handle)

    def device_info(self):
        name = C.create_string_buffer(256)
        cus = C.c_int32()
        _lib.check(self.lib.rf_ctx_device_info(self.handle, name, 256, C.byref(cus)))
        return name.value.decode(), cus.value

    # ledger (MemoryBudget on the device domain)
    @property
    def vram_used(self) -> int:
        return self.lib.rf_vram_used(self.handle)

    @property
    def vram_total(self) -> int:
        return self.lib.rf_vram_total(self.handle)

    @property
    def vram_peak(self) -> int:
        return self.lib.rf_vram_peak(self.handle)

    def charge(self, name: str) -> Optional[int]:
        v = C.c_uint64()
        rc = self.lib.rf_vram_charge(self.handle, name.encode(), C.byref(v))
        return v.value if rc == _lib.RF_OK else None

    def rename_prefix(self, old: str, new: str) -> None:
        _lib.check(self.lib.rf_vram_rename_prefix(self.handle, old.encode(), new.encode()))

    # rf_matvec's repack cache (off by default)
    def matvec_cache(self, max_bytes: int) -> None:
        """Keep packed copies of the GGUF tensors matvec() is handed, up to
        max_bytes (0 turns the cache off and frees it).  The tensors' bytes
        must not change while cached (see matvec_cache_forget)."""
        _lib.check(self.lib.rf_matvec_cache(self.handle, int(max_bytes)))

    def matvec_cache_forget(self, w, nbytes: Optional[int] = None) -> None:
        """Drop the cached copies of every tensor whose bytes overlap w's."""
        n = w.nbytes if (nbytes is None and isinstance(w, DeviceArray)) else int(nbytes or 0)
        _lib.check(self.lib.rf_matvec_cache_forget(self.handle, _ptr(w), n))

    def matvec_cache_stats(self) -> dict:
        v = [C.c_uint64() for _ in range(4)]
        _lib.check(self.lib.rf_matvec_cache_stats(self.handle, *(C.byref(x) for x in v)))
        return dict(zip(("entries", "bytes", "hits", "misses"), (x.value for x in v)))

    # buffers
    def alloc(self, nbytes: int, charge: Optional[str] = None, shape=None, dtype=np.uint8) -> DeviceArray:
        if charge is None:
            Context._serial += 1
            charge = f"tmp:array:{Context._serial}"
        if shape is None:
            shape = (int(nbytes) // np.dtype(dtype).itemsize,)
        elif int(np.prod(shape)) * np.dtype(dtype).itemsize > int(nbytes):
            raise ValueError(f"shape {tuple(shape)} of {np.dtype(dtype)} exceeds {int(nbytes)} bytes")
        p = C.c_void_p()
        _lib.check(self.lib.rf_vram_alloc(self.handle, charge.encode(), int(nbytes), C.byref(p)))
        return DeviceArray(self, p.value, int(nbytes), shape, dtype, charge)

    def empty(self, shape, dtype=np.float32, charge: Optional[str] = None) -> DeviceArray:
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return self.alloc(max(n, 1), charge, shape, dtype)

    def array(self, host: np.ndarray, charge: Optional[str] = None) -> DeviceArray:
        h = np.ascontiguousarray(host)
        d = self.alloc(max(h.nbytes, 1), charge, h.shape, h.dtype)
        if h.nbytes:
            d.upload(h)
        return d

    # synthetic payloads (bench / test inputs)
    def synth_blocks(self, ggml_type: int, seed: int, first_block: int, n_blocks: int, scale_mul: float,
                     dst: DeviceArray, stream=None) -> None:
        _lib.check(self.lib.rf_synth_blocks(self.handle, ggml_type, seed, first_block, n_blocks, scale_mul,
                                            _ptr(dst), dst.nbytes, stream))

    # events
    def copy(self, dst, src, nbytes: int, stream=None) -> None:
        """Device-to-device copy (hipMemcpyAsync on `stream`, default the compute stream)."""
        _lib.check(self.lib.rf_copy_async(self.handle, _ptr(dst), _ptr(src), nbytes, stream))

    def capture(self):
        """Context manager: the calls enqueued on the compute stream inside the
        block are recorded into a graph (CapturedGraph) instead of running."""
        return _Capture(self)

    def event(self):
        e = C.c_void_p()
        _lib.check(self.lib.rf_event_create(self.handle, C.byref(e)))
        return e.value

    def record(self, ev, stream=None) -> None:
        _lib.check(self.lib.rf_event_record(self.handle, ev, stream))

    def elapsed_ms(self, a, b) -> float:
        ms = C.c_float()
        _lib.check(self.lib.rf_event_synchronize(self.handle, b))
        _lib.check(self.lib.rf_event_elapsed_ms(self.handle, a, b, C.byref(ms)))
        return ms.value

    def destroy_event(self, ev) -> None:
        _lib.check(self.lib.rf_event_destroy(self.handle, ev))


# --------------------------------------------------------------------- ops

def _fits(op: str, **need) -> None:
    """Raise the reference's shape-mismatch error when a DeviceArray argument
    holds fewer bytes than the call reads or writes (raw device addresses are
    passed through unchecked: their sizes are unknown here)."""
    for name, (arr, nbytes) in need.items():
        if isinstance(arr, DeviceArray) and arr.nbytes < nbytes:
            raise RamforgeError(_lib.RF_ERR_INVALID,
                                f"{op} shape mismatch: {name} holds {arr.nbytes} bytes, {nbytes} needed")


def _rows(out_dim: int, row_start: int, row_count: Optional[int]) -> int:
    return max(0, out_dim - row_start) if row_count is None else row_count


def _fits_matvec(w_shape, x, y, rows: int) -> None:
    """The reference's first matvec check, x / y lengths against the shape
    (quant.rs:990-997), on DeviceArray capacities."""
    out_dim, in_dim = w_shape
    xl = x.nbytes // 4 if isinstance(x, DeviceArray) else None
    yl = y.nbytes // 4 if isinstance(y, DeviceArray) else None
    if (xl is not None and xl < in_dim) or (yl is not None and yl < rows):
        raise RamforgeError(_lib.RF_ERR_INVALID, f"matvec shape mismatch: W {[out_dim, in_dim]}, x {xl}, y {yl}")


def matvec(ctx: Context, ggml_type: int, w, w_shape: Sequence[int], x, y, row_start: int = 0,
           row_count: Optional[int] = None, w_bytes: Optional[int] = None, stream=None) -> None:
    """quant::matvec_<fmt>_row_range (quant.rs:913-975): kernel shape
    ``w_shape = [out_dim, in_dim]``; y is local to ``row_start``."""
    if len(w_shape) != 2:
        raise RamforgeError(_lib.RF_ERR_INVALID, f"{GGML.NAMES.get(ggml_type, ggml_type)} matvec expects 2D weight")
    out_dim, in_dim = (int(v) for v in w_shape)
    _fits_matvec((out_dim, in_dim), x, y, _rows(out_dim, row_start, row_count))
    wb = w.nbytes if (w_bytes is None and isinstance(w, DeviceArray)) else int(w_bytes or 0)
    rc = ctx.lib.rf_matvec(ctx.handle, ggml_type, _ptr(w), wb, out_dim, in_dim, _ptr(x), _ptr(y), row_start,
                           RF_ALL_ROWS if row_count is None else row_count, stream)
    _lib.check(rc)


def packed_supported(ggml_type: int, in_dim: int) -> bool:
    """Whether the packed (device-native) layout and kernel cover (type, in_dim)."""
    return bool(_lib.load().rf_packed_supported(ggml_type, in_dim))


def pack_weights(ctx: Context, ggml_type: int, raw, rows: int, in_dim: int, packed, raw_bytes: Optional[int] = None,
                 stream=None) -> None:
    """GGUF Q8_0 / Q4_0 / Q4_K / Q6_K payload [rows][in_dim] -> packed layout:
    the byte ranges of each block split into regions stored for all rows
    (Q8_0 / Q4_0: codes, f16 scales; Q4_K: codes, 16-byte headers; Q6_K: ql,
    qh, scales, d); same byte count."""
    rb = raw.nbytes if (raw_bytes is None and isinstance(raw, DeviceArray)) else int(raw_bytes or 0)
    pb = packed.nbytes if isinstance(packed, DeviceArray) else rb
    _lib.check(ctx.lib.rf_pack_weights(ctx.handle, ggml_type, _ptr(raw), rb, rows, in_dim, _ptr(packed), pb, stream))


def matvec_packed(ctx: Context, ggml_type: int, w, w_shape: Sequence[int], x, y, row_start: int = 0,
                  row_count: Optional[int] = None, w_bytes: Optional[int] = None, stream=None) -> None:
    """matvec() on a packed tensor (see pack_weights)."""
    if len(w_shape) != 2:
        raise RamforgeError(_lib.RF_ERR_INVALID, f"{GGML.NAMES.get(ggml_type, ggml_type)} matvec expects 2D weight")
    out_dim, in_dim = (int(v) for v in w_shape)
    _fits_matvec((out_dim, in_dim), x, y, _rows(out_dim, row_start, row_count))
    wb = w.nbytes if (w_bytes is None and isinstance(w, DeviceArray)) else int(w_bytes or 0)
    rc = ctx.lib.rf_matvec_packed(ctx.handle, ggml_type, _ptr(w), wb, out_dim, in_dim, _ptr(x), _ptr(y), row_start,
                                  RF_ALL_ROWS if row_count is None else row_count, stream)
    _lib.check(rc)


def matmul_packed(ctx: Context, ggml_type: int, w, w_shape: Sequence[int], x, n_tokens: int, y,
                  w_bytes: Optional[int] = None, stream=None) -> None:
    """Batched matvec for prompt prefill: y[t] = W x[t] for n_tokens rows of
    x ([n_tokens][in_dim]) on a packed tensor, y [n_tokens][out_dim], on the
    matrix cores (no reference counterpart: the reference runs matvec_<fmt>
    per prompt token, quant.rs:898-1327)."""
    if len(w_shape) != 2:
        raise RamforgeError(_lib.RF_ERR_INVALID, f"{GGML.NAMES.get(ggml_type, ggml_type)} matmul expects 2D weight")
    out_dim, in_dim = (int(v) for v in w_shape)
    _fits("matmul", x=(x, 4 * n_tokens * in_dim), y=(y, 4 * n_tokens * out_dim))
    wb = w.nbytes if (w_bytes is None and isinstance(w, DeviceArray)) else int(w_bytes or 0)
    _lib.check(ctx.lib.rf_matmul_packed(ctx.handle, ggml_type, _ptr(w), wb, out_dim, in_dim, _ptr(x), n_tokens,
                                        _ptr(y), stream))


def dequantize_rows(ctx: Context, ggml_type: int, w, in_dim: int, row_start: int, row_count: int, out,
                    w_bytes: Optional[int] = None, stream=None) -> None:
    """dequantize_row_<fmt> (quant.rs:615-868) for a row range, bit-exact."""
    _fits("row decode", out=(out, 4 * row_count * in_dim))
    wb = w.nbytes if (w_bytes is None and isinstance(w, DeviceArray)) else int(w_bytes or 0)
    _lib.check(ctx.lib.rf_dequantize_rows(ctx.handle, ggml_type, _ptr(w), wb, in_dim, row_start, row_count,
                                          _ptr(out), stream))


def attention_checked(ctx: Context, q, k_hist, v_hist, k_new, v_new, hist_len: int, n_heads: int,
                      n_kv_heads: int, head_dim: int, out: Optional[DeviceArray] = None, stream=None) -> DeviceArray:
    """ops::attention_checked (ops.rs:49-69) -> compute::attention_reference."""
    qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
    _fits("attention tensor", q=(q, 4 * qd), k_hist=(k_hist, 4 * hist_len * kvd), v_hist=(v_hist, 4 * hist_len * kvd),
          k_new=(k_new, 4 * kvd), v_new=(v_new, 4 * kvd), out=(out, 4 * qd))
    if out is None:
        out = ctx.empty((qd,))
    _lib.check(ctx.lib.rf_attention_decode(ctx.handle, _ptr(q), _ptr(k_hist), _ptr(v_hist), _ptr(k_new),
                                           _ptr(v_new), hist_len, n_heads, n_kv_heads, head_dim, _ptr(out), stream))
    return out


def attention_checked_noalloc(ctx: Context, q, k_hist, v_hist, k_new, v_new, hist_len: int, n_heads: int,
                              n_kv_heads: int, head_dim: int, out: DeviceArray, stream=None) -> DeviceArray:
    """attention_checked through rf_attention_decode_noalloc: the split
    records live in the library's static per-device scratch array, so the
    call allocates nothing (the caller passes ``out``)."""
    qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
    _fits("attention tensor", q=(q, 4 * qd), k_hist=(k_hist, 4 * hist_len * kvd), v_hist=(v_hist, 4 * hist_len * kvd),
          k_new=(k_new, 4 * kvd), v_new=(v_new, 4 * kvd), out=(out, 4 * qd))
    _lib.check(ctx.lib.rf_attention_decode_noalloc(ctx.handle, _ptr(q), _ptr(k_hist), _ptr(v_hist), _ptr(k_new),
                                                   _ptr(v_new), hist_len, n_heads, n_kv_heads, head_dim, _ptr(out),
                                                   stream))
    return out


def apply_rope(ctx: Context, q, k, pos: int, head_dim: int, n_heads: int, n_kv_heads: int, freq_base: float,
               stream=None) -> None:
    """ops::apply_rope (ops.rs:9-20): half-split RoPE in place."""
    _fits("RoPE", q=(q, 4 * n_heads * head_dim), k=(k, 4 * n_kv_heads * head_dim))
    _lib.check(ctx.lib.rf_rope(ctx.handle, _ptr(q), _ptr(k), pos, head_dim, n_heads, n_kv_heads, freq_base, stream))


def rmsnorm(ctx: Context, x, weight, n: int, eps: float, out, stream=None) -> None:
    _fits("RMSNorm", input=(x, 4 * n), weight=(weight, 4 * n), output=(out, 4 * n))
    _lib.check(ctx.lib.rf_rmsnorm(ctx.handle, _ptr(x), _ptr(weight), n, eps, _ptr(out), stream))


def add(ctx: Context, a, b, n: int, out, stream=None) -> None:
    _fits("elementwise", a=(a, 4 * n), b=(b, 4 * n), out=(out, 4 * n))
    _lib.check(ctx.lib.rf_add(ctx.handle, _ptr(a), _ptr(b), n, _ptr(out), stream))


def bias_add(ctx: Context, v, bias, n: int, stream=None) -> None:
    """v += bias in place (model_executor.rs:161-194, the Q/K/V bias step)."""
    _fits("bias add", v=(v, 4 * n), bias=(bias, 4 * n))
    _lib.check(ctx.lib.rf_bias_add(ctx.handle, _ptr(v), _ptr(bias), n, stream))


def mul(ctx: Context, a, b, n: int, out, stream=None) -> None:
    _fits("elementwise", a=(a, 4 * n), b=(b, 4 * n), out=(out, 4 * n))
    _lib.check(ctx.lib.rf_mul(ctx.handle, _ptr(a), _ptr(b), n, _ptr(out), stream))


def silu(ctx: Context, x, n: int, out, stream=None) -> None:
    _fits("SiLU", x=(x, 4 * n), out=(out, 4 * n))
    _lib.check(ctx.lib.rf_silu(ctx.handle, _ptr(x), n, _ptr(out), stream))


def swiglu(ctx: Context, gate, up, n: int, out, stream=None) -> None:
    _fits("elementwise", gate=(gate, 4 * n), up=(up, 4 * n), out=(out, 4 * n))
    _lib.check(ctx.lib.rf_swiglu(ctx.handle, _ptr(gate), _ptr(up), n, _ptr(out), stream))


def softmax(ctx: Context, values, n: int, stream=None) -> None:
    _fits("softmax", values=(values, 4 * n))
    _lib.check(ctx.lib.rf_softmax(ctx.handle, _ptr(values), n, stream))


def argmax(ctx: Context, logits, n: int, out_index, stream=None) -> None:
    """Greedy Sampler::sample_checked (sampling.rs:45-57) into device memory."""
    _fits("argmax", logits=(logits, 4 * n), out_index=(out_index, 4))
    _lib.check(ctx.lib.rf_argmax(ctx.handle, _ptr(logits), n, _ptr(out_index), stream))


# ------------------------------------------------- backend / dispatch mirror

@dataclass
class GpuTensor:
    """A TensorData held in VRAM (core/src/tensor.rs:328-343): raw GGUF
    payload with ggml shape ``[in, out]``."""

    ggml_type: int
    shape: tuple
    data: DeviceArray


class GpuBackend:
    """ComputeBackend (runtime/src/backend.rs:27-52) over device buffers."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    def name(self) -> str:
        return "HIP-gfx950"

    def num_threads(self) -> int:
        return 1  # parallelism is inside the kernels; calls come from one thread

    def matvec(self, w: DeviceArray, w_shape: Sequence[int], x: DeviceArray, y: DeviceArray) -> None:
        """F32 matvec with ``w_shape = [in, out]`` (ggml layout)."""
        if len(w_shape) != 2:
            raise RamforgeError(_lib.RF_ERR_INVALID,
                                f"backend matvec expects 2D w_shape [in, out] (ggml layout), got {list(w_shape)}")
        in_dim, out_dim = int(w_shape[0]), int(w_shape[1])
        if x.shape[0] != in_dim or y.shape[0] != out_dim or w.nbytes < 4 * in_dim * out_dim:
            raise RamforgeError(
                _lib.RF_ERR_INVALID,
                f"backend matvec arity mismatch (ggml layout [in, out]): shape {list(w_shape)} implies in={in_dim}, "
                f"out={out_dim}, but got w bytes={w.nbytes}, x.len()={x.shape[0]}, y.len()={y.shape[0]}")
        matvec(self.ctx, GGML.F32, w, (out_dim, in_dim), x, y)

    def rmsnorm(self, x, weight, eps: float, y) -> None:
        rmsnorm(self.ctx, x, weight, x.shape[0], eps, y)

    def add(self, a, b, out) -> None:
        add(self.ctx, a, b, a.shape[0], out)

    def mul(self, a, b, out) -> None:
        mul(self.ctx, a, b, a.shape[0], out)

    def silu(self, x, out) -> None:
        silu(self.ctx, x, x.shape[0], out)

    def softmax(self, x) -> None:
        softmax(self.ctx, x, x.shape[0])


def matvec_backend(backend: GpuBackend, td: GpuTensor, x: DeviceArray, y: DeviceArray) -> None:
    """compute_dispatch::matvec_backend (compute_dispatch.rs:40-58): F32 goes
    through the backend matvec, quantized tensors through the block kernels
    after the ``[in, out] -> [out, in]`` flip (compute_dispatch.rs:109-110)."""
    if len(td.shape) != 2:
        raise RamforgeError(_lib.RF_ERR_INVALID,
                            f"{GGML.NAMES.get(td.ggml_type)} matvec expects 2D tensor shape, got {list(td.shape)}")
    if td.ggml_type == GGML.F32:
        backend.matvec(td.data, td.shape, x, y)
        return
    in_dim, out_dim = td.shape
    if x.shape[0] != in_dim or y.shape[0] != out_dim:
        raise RamforgeError(_lib.RF_ERR_INVALID,
                            f"matvec shape mismatch: W {[out_dim, in_dim]}, x {x.shape[0]}, y {y.shape[0]}")
    matvec(backend.ctx, td.ggml_type, td.data, (out_dim, in_dim), x, y)


# ------------------------------------------------------------------- model

class ByteSource:
    """Byte source for streamed layers (rf_read_fn): a file read with
    os.preadv straight into the pinned staging buffer, or an in-memory buffer.
    ``fail_at`` (an offset) makes reads that cover it fail, for tests of the
    error path."""

    def __init__(self, path_or_buffer):
        self.fd = None
        self.buf = None
        if isinstance(path_or_buffer, (str, os.PathLike)):
            self.fd = os.open(path_or_buffer, os.O_RDONLY)
        else:
            self.buf = np.frombuffer(path_or_buffer, np.uint8)
        self.fail_at = None
        self.calls = 0
        self.callback = _lib.READ_FN(self._read)

    def _read(self, _user, offset, length, dst):
        self.calls += 1
        try:
            if self.fail_at is not None and offset <= self.fail_at < offset + length:
                return 5
            if self.buf is not None:
                if offset + length > self.buf.size:
                    return 1
                C.memmove(dst, self.buf.ctypes.data + offset, length)
                return 0
            view = memoryview((C.c_char * length).from_address(dst)).cast("B")
            got = 0
            while got < length:
                n = os.preadv(self.fd, [view[got:]], offset + got)
                if n <= 0:
                    return 2
                got += n
            return 0
        except Exception:  # reported to the library as a failed read
            return 3

    def close(self) -> None:
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None


class FileSource:
    """Byte source over a model file read by the library itself
    (rf_file_source_read: each range split over `threads` pread loops), for
    GpuLlamaModel.set_reader."""

    def __init__(self, path, threads: int = 8):
        self.lib = _lib.load()
        h = C.c_void_p()
        _lib.check(self.lib.rf_file_source_open(os.fsencode(path), threads, C.byref(h)))
        self.handle = h.value
        # the library's own rf_read_fn, called with the handle as `user`
        self.callback = _lib.READ_FN(C.cast(self.lib.rf_file_source_read, C.c_void_p).value)
        self.user = self.handle

    def close(self) -> None:
        if self.handle:
            self.lib.rf_file_source_close(self.handle)
            self.handle = None


class GpuLlamaModel:
    """VRAM-resident dense llama decoder (rf_model_* in the C ABI)."""

    def __init__(self, ctx: Context, cfg: dict, kv_capacity: Optional[int] = None, kv_initial: Optional[int] = None):
        """kv_initial: allocate the KV cache for that many positions and grow it
        in 256-position chunks up to kv_capacity (rf_model_create_growing)."""
        self.ctx = ctx
        self.cfg = dict(cfg)
        c = ModelConfig(**{k: self.cfg[k] for k, _ in ModelConfig._fields_})
        self._c = c
        h = C.c_void_p()
        cap = int(kv_capacity if kv_capacity is not None else cfg["context_length"])
        if kv_initial is None:
            _lib.check(ctx.lib.rf_model_create(ctx.handle, C.byref(c), cap, C.byref(h)))
        else:
            _lib.check(ctx.lib.rf_model_create_growing(ctx.handle, C.byref(c), cap, int(kv_initial), C.byref(h)))
        self.handle = h
        self.kv_capacity = cap

    def close(self) -> None:
        if self.handle:
            self.ctx.lib.rf_model_destroy(self.handle)
            self.handle = None

    def enable_streaming(self, layer_cache_bytes: int) -> None:
        """Keep block tensors in pinned host memory and stream layers into an
        LRU device cache of at most layer_cache_bytes (call before loading)."""
        _lib.check(self.ctx.lib.rf_model_enable_streaming(self.handle, int(layer_cache_bytes)))

    def set_cache_policy(self, policy: int) -> None:
        """0: least recently used (reference LayerCache); 1: next use in the layer cycle."""
        _lib.check(self.ctx.lib.rf_model_set_cache_policy(self.handle, policy))

    def set_stream_units(self, per_layer: int) -> None:
        """Streaming units per layer (rf_model_set_stream_units): 1 the whole
        layer (default); 2 attention tensors with the norms | gate, up,
        down; 3 attention | gate, up | down.  Units are loaded, cached and
        evicted separately."""
        _lib.check(self.ctx.lib.rf_model_set_stream_units(self.handle, int(per_layer)))

    def set_reader(self, source: "ByteSource", staging_bytes: int = 64 << 20) -> None:
        """Streamed layers read their declared tensors from `source`
        (rf_model_set_reader); call after enable_streaming."""
        self._source = source  # keeps the callback alive
        _lib.check(self.ctx.lib.rf_model_set_reader(self.handle, source.callback, getattr(source, "user", None),
                                                    int(staging_bytes)))

    def set_read_ahead(self, on: bool) -> None:
        """Read the next layer the pass will load from the byte source on a
        worker thread (rf_model_set_read_ahead; the reader must then be
        thread-safe; on by default for FileSource, off for ByteSource)."""
        _lib.check(self.ctx.lib.rf_model_set_read_ahead(self.handle, int(bool(on))))

    def set_tensor_source(self, name: str, ggml_type: int, ne0: int, ne1: int, offset: int, nbytes: int) -> None:
        """Declare block tensor `name` at [offset, offset + nbytes) of the byte source."""
        _lib.check(self.ctx.lib.rf_model_set_tensor_source(self.handle, name.encode(), ggml_type, ne0, ne1,
                                                           int(offset), int(nbytes)))

    def set_persistent_policy(self, policy: int) -> None:
        """0: token_embd / output resident when at most 25% of the budget, else
        streamed from mapped pinned host memory; 1: always streamed; 2: always
        resident; 3: token_embd always streamed, output by the 25% rule
        (streaming models only; before those tensors load)."""
        _lib.check(self.ctx.lib.rf_model_set_persistent_policy(self.handle, policy))

    def persistent_streamed(self) -> dict:
        v = C.c_uint32()
        _lib.check(self.ctx.lib.rf_model_persistent_streamed(self.handle, C.byref(v)))
        return {"token_embd": bool(v.value & 1), "output": bool(v.value & 2)}

    def profile(self, enable: bool) -> None:
        """Bracket every launch group of the following eager forwards with HIP
        events (rf_model_profile)."""
        _lib.check(self.ctx.lib.rf_model_profile(self.handle, 1 if enable else 0))

    def profile_read(self, reset: bool = False) -> dict:
        """{group: (device ms, launches)} accumulated by the forward profiler."""
        ms, n = (C.c_double * 6)(), (C.c_uint64 * 6)()
        _lib.check(self.ctx.lib.rf_model_profile_read(self.handle, ms, n, 1 if reset else 0))
        return {k: (ms[v - 1], int(n[v - 1])) for k, v in self.KERNELS.items()}

    def read_stats(self) -> dict:
        out = (C.c_uint64 * 2)()
        _lib.check(self.ctx.lib.rf_model_read_stats(self.handle, out))
        return {"calls": int(out[0]), "bytes": int(out[1])}

    def host_bytes(self) -> int:
        """Pinned host bytes the model holds (streamed tensors' host copies,
        mapped persistent weights, the byte source's staging buffers)."""
        v = C.c_uint64()
        _lib.check(self.ctx.lib.rf_model_host_bytes(self.handle, C.byref(v)))
        return v.value

    def residency_stats(self) -> dict:
        out = (C.c_uint64 * 6)()
        _lib.check(self.ctx.lib.rf_model_residency_stats(self.handle, out))
        keys = ("hits", "misses", "evictions", "uploaded_bytes", "cached_bytes", "cached_layers")
        return dict(zip(keys, (int(v) for v in out)))

    def set_tensor(self, name: str, ggml_type: int, ne0: int, ne1: int, data: np.ndarray) -> None:
        h = np.ascontiguousarray(data)
        _lib.check(self.ctx.lib.rf_model_set_tensor(self.handle, name.encode(), ggml_type, ne0, ne1,
                                                    h.ctypes.data, h.nbytes))

    def synth_tensor(self, name: str, ggml_type: int, ne0: int, ne1: int, seed: int, scale_mul: float,
                     constant: float = float("nan")) -> None:
        _lib.check(self.ctx.lib.rf_model_synth_tensor(self.handle, name.encode(), ggml_type, ne0, ne1, seed,
                                                      scale_mul, constant))

    def reset(self) -> None:
        _lib.check(self.ctx.lib.rf_model_reset(self.handle))

    @property
    def seq_len(self) -> int:
        return self.ctx.lib.rf_model_seq_len(self.handle)

    def forward(self, token: int, pos: int, want_hidden: bool = False) -> Optional[np.ndarray]:
        hidden = np.empty(self.cfg["embedding_length"], np.float32) if want_hidden else None
        _lib.check(self.ctx.lib.rf_model_forward(self.handle, token, pos,
                                                 hidden.ctypes.data if hidden is not None else None))
        return hidden

    def prefill(self, tokens: Sequence[int], want_hidden: bool = False) -> Optional[np.ndarray]:
        """Forwards tokens at positions seq_len.. as batched chunks (same
        result as one forward() per token, to f32 accuracy)."""
        p = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        hidden = np.empty(self.cfg["embedding_length"], np.float32) if want_hidden else None
        _lib.check(self.ctx.lib.rf_model_prefill(self.handle, p.ctypes.data, len(p),
                                                 hidden.ctypes.data if hidden is not None else None))
        return hidden

    def set_prefill(self, batched: bool) -> None:
        """generate() forwards its prompt batched (True) or token by token."""
        _lib.check(self.ctx.lib.rf_model_set_prefill(self.handle, 1 if batched else 0))

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg["vocab_size"], np.float32)
        _lib.check(self.ctx.lib.rf_model_logits(self.handle, out.ctypes.data))
        return out

    def generate(self, prompt: Sequence[int], max_tokens: int, eos: int = -1) -> list:
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        out = np.zeros(max(max_tokens, 1), np.uint32)
        n = C.c_uint64()
        _lib.check(self.ctx.lib.rf_model_generate(self.handle, p.ctypes.data, len(p), max_tokens, eos,
                                                  out.ctypes.data, C.byref(n)))
        return [int(t) for t in out[: n.value]]

    def use_graph(self, enable: bool) -> None:
        _lib.check(self.ctx.lib.rf_model_use_graph(self.handle, 1 if enable else 0))

    def kv_growth(self, initial_tokens: int) -> None:
        """Start the (empty) KV cache at initial_tokens positions and grow it in
        256-position chunks as positions are needed (KvCache::grow_to_with_budget)."""
        _lib.check(self.ctx.lib.rf_model_kv_growth(self.handle, initial_tokens))

    def kv_positions(self) -> int:
        """Positions the KV cache holds now (KvCache::capacity_tokens); at most kv_capacity."""
        n = C.c_uint64()
        _lib.check(self.ctx.lib.rf_model_kv_capacity(self.handle, C.byref(n)))
        return n.value

    def decode_steps(self, steps: int) -> None:
        _lib.check(self.ctx.lib.rf_model_decode_steps(self.handle, steps))

    def paths(self, pos: int = 0) -> dict:
        """Which kernels run: the split-K attention kernel (else the any-shape
        one), its launch regime for a decode step at `pos`, and whether
        prefill is batched (else one forward per token)."""
        sa, rg, bp = C.c_int32(), C.c_int32(), C.c_int32()
        _lib.check(self.ctx.lib.rf_model_paths(self.handle, pos, C.byref(sa), C.byref(rg), C.byref(bp)))
        return {"split_attention": bool(sa.value), "regime": rg.value, "batched_prefill": bool(bp.value)}

    KERNELS = {"qkv": 1, "attention": 2, "oproj": 3, "gateup": 4, "down": 5, "logits": 6}

    def time_kernel(self, kind: str, reps: int = 1):
        """(avg ms per launch, algorithmic bytes per launch, launches) of one
        decode-step launch group, timed with HIP events on the compute stream."""
        ms, b, n = C.c_float(), C.c_uint64(), C.c_uint64()
        _lib.check(self.ctx.lib.rf_model_time_kernel(self.handle, self.KERNELS[kind], reps, C.byref(ms), C.byref(b),
                                                     C.byref(n)))
        return ms.value, b.value, n.value

    def kernel_name(self, kind: str) -> str:
        """The packed matvec kernel instance a launch group runs, as the
        profiler's kernel trace names it ("" for none)."""
        buf = C.create_string_buffer(256)
        _lib.check(self.ctx.lib.rf_model_kernel_name(self.handle, self.KERNELS[kind], buf, 256))
        return buf.value.decode()

    def read_tokens(self, n: int) -> list:
        out = np.zeros(max(n, 1), np.uint32)
        _lib.check(self.ctx.lib.rf_model_read_tokens(self.handle, out.ctypes.data, n))
        return [int(t) for t in out[:n]]


def tune_matvec_tile_bytes(nbytes: int = 0) -> int:
    """Set (nbytes > 0) and return the LDS bytes per one-shot matvec tile."""
    return _lib.load().rf_tune_matvec_tile_bytes(nbytes)


def tune_matvec_kernel(mode: int = -1) -> int:
    """GGUF-layout matvec kernels: 2 (default) plain Q8_0 / Q4_0 / Q6_K
    matvecs (Q4_K up to 4096 inputs) stage each row per wavefront in LDS
    through 16-byte loads, plain F32 ones load rows per wavefront into
    registers, the rest as 1; 1 persistent streaming kernel with LDS row
    tiles; 0 one-shot tile kernel; -1 queries.  Returns the mode in effect."""
    return _lib.load().rf_tune_matvec_kernel(mode)


def tune_matvec_digits(mode: int = -1) -> int:
    """0: float x everywhere (default); 1: packed Q8_0 / Q4_0 launches with
    >= 24 KiB of codes per wavefront take x as int8 digit planes (30 bits
    below each 16-element unit's largest element); 2: every launch whose LDS
    holds them; -1 queries.  Returns the mode in effect."""
    return _lib.load().rf_tune_matvec_digits(mode)


def tune_packed_inflight(mode: int = -1) -> int:
    """1: packed launches whose rows fit one step, with a wavefront per row,
    request the row before staging x (default), 0: the two-step ring; -1
    queries.  Same results either way."""
    return _lib.load().rf_tune_packed_inflight(mode)


def tune_attention_merge(mode: int = -1) -> int:
    """1: in decode steps whose attention splits per query head, the
    o-projection merges the attention's chunk records while staging its x
    (no merge kernel; default), 0: the merge kernel, then the o-projection;
    -1 queries.  The two differ in rounding only.  Returns the mode in
    effect."""
    return _lib.load().rf_tune_attention_merge(mode)


def tune_attention_kernel(mode: int = -1) -> int:
    """Decode-step attention: the one-pass online-softmax kernel for launches
    per query head (1, default), for every launch (2) or none (0: two-pass,
    scores in LDS, then V); -1 queries.  Batched prefill keeps the two-pass
    kernel.  Returns the mode in effect."""
    return _lib.load().rf_tune_attention_kernel(mode)


def tune_attention_single(positions: int = -1) -> int:
    """Longest context (64, 128 or 256) decode attention serves with one
    chunk per query head and no merge; -1 queries.  Returns the value in
    effect."""
    return _lib.load().rf_tune_attention_single(positions)


def tune_prefill_attention(mode: int = -1) -> int:
    """Batched-prefill attention on the matrix-core kernel (16-token tiles,
    each K / V row read once per tile) past 1024 positions (1, default), for
    every chunk (2), or never (0: the decode split kernel with a token
    dimension); -1 queries.  They differ in rounding only.  Returns the mode
    in effect."""
    return _lib.load().rf_tune_prefill_attention(mode)


def tune_packed_weights(mode: int = -1) -> int:
    """1: Q8_0 / Q4_0 / Q4_K / Q6_K projection weights of models are repacked
    into the device-native layout at install (default; the batched prefill
    needs it), 0: kept as GGUF bytes; -1 queries.  Returns the mode in
    effect."""
    return _lib.load().rf_tune_packed_weights(mode)


# Fail loudly at import if the HIP library was not built.
_lib.load()
