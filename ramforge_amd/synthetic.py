"""Random-init llama models and matvec inputs for the benchmark configurations.

The payloads come from the seeded counter generator (rf_synth_blocks on the
device; the CPU oracle carries a byte-identical copy), so a model can be built
directly in VRAM in milliseconds and rebuilt bit-for-bit on the host for the
CPU baseline and the parity tests.

Scale fields are f16(|n| * scale_mul) with n ~ Irwin-Hall(12) (a normal
approximation that is exact in binary64 on both sides).
"""
from __future__ import annotations

from dataclasses import dataclass

# ggml type ids (core/src/types.rs:238-292)
F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14

# Per-format scale multipliers: Q8_0 d = |N(0,0.02)|/127,
# which gives decoded weights of standard deviation 0.0117; the others are
# set so that their decoded weights have that same spread (measured through
# the reference's decode, whose f16 subnormal rule halves most of the small
# K-quant scales).  With weights several times smaller, a random model's
# layers barely move the residual stream and greedy decoding repeats one
# token.
SCALE_MUL = {Q8_0: 0.02 / 127.0, Q4_0: 0.02 / 8.0, Q4_K: 5.07e-5, Q6_K: 1.71e-5, F32: 0.02}

# BASELINE.json configurations
CONFIG_4 = dict(vocab_size=32000, context_length=4096, embedding_length=2048, block_count=16,
                feed_forward_length=8192, head_count=32, head_count_kv=8, head_dim=64, rms_eps=1e-5,
                rope_freq_base=10000.0)
CONFIG_8B = dict(vocab_size=128256, context_length=8192, embedding_length=4096, block_count=32,
                 feed_forward_length=14336, head_count=32, head_count_kv=8, head_dim=128, rms_eps=1e-5,
                 rope_freq_base=10000.0)


@dataclass
class TensorSpec:
    name: str
    ggml_type: int
    ne0: int          # ggml [in, out]
    ne1: int
    seed: int
    scale_mul: float
    constant: float = float("nan")  # F32 constant fill (norm weights)


def llama_specs(cfg: dict, body_type: int = Q8_0, output_type: int | None = None, embd_type: int | None = None,
                seed: int = 1234) -> list[TensorSpec]:
    """GGUF tensor list of a random-init llama model."""
    out_t = body_type if output_type is None else output_type
    emb_t = body_type if embd_type is None else embd_type
    d, f, V = cfg["embedding_length"], cfg["feed_forward_length"], cfg["vocab_size"]
    qd = cfg["head_count"] * cfg["head_dim"]
    kvd = cfg["head_count_kv"] * cfg["head_dim"]
    specs = []
    k = 0

    def add(name, t, ne0, ne1, const=float("nan")):
        nonlocal k
        k += 1
        specs.append(TensorSpec(name, t, ne0, ne1, seed * 1000003 + k, SCALE_MUL.get(t, 0.02), const))

    add("token_embd.weight", emb_t, d, V)
    add("output_norm.weight", F32, d, 1, 1.0)
    add("output.weight", out_t, d, V)
    for i in range(cfg["block_count"]):
        add(f"blk.{i}.attn_norm.weight", F32, d, 1, 1.0)
        add(f"blk.{i}.attn_q.weight", body_type, d, qd)
        add(f"blk.{i}.attn_k.weight", body_type, d, kvd)
        add(f"blk.{i}.attn_v.weight", body_type, d, kvd)
        add(f"blk.{i}.attn_output.weight", body_type, qd, d)
        add(f"blk.{i}.ffn_norm.weight", F32, d, 1, 1.0)
        add(f"blk.{i}.ffn_gate.weight", body_type, d, f)
        add(f"blk.{i}.ffn_up.weight", body_type, d, f)
        add(f"blk.{i}.ffn_down.weight", body_type, f, d)
    return specs


def n_blocks(spec: TensorSpec) -> int:
    qk = 1 if spec.ggml_type == F32 else (32 if spec.ggml_type in (Q4_0, Q8_0, 6) else 256)
    return spec.ne0 // qk * spec.ne1


def weight_bytes(specs: list[TensorSpec]) -> int:
    geo = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
    tot = 0
    for s in specs:
        qk, bs = geo[s.ggml_type]
        tot += s.ne0 // qk * bs * s.ne1
    return tot


def build_device_model(ctx, cfg: dict, specs: list[TensorSpec], kv_capacity: int,
                       stream_cache_bytes: int | None = None, cache_policy: int = 0, kv_initial: int | None = None,
                       persistent_policy: int = 0):
    """A GpuLlamaModel with every tensor generated on the device.  With
    stream_cache_bytes the block tensors go to pinned host memory and layers
    stream through a device LRU cache of that many bytes (cache_policy 1:
    next-use eviction; persistent_policy: where the embedding and output
    projection live, see GpuLlamaModel.set_persistent_policy); with
    kv_initial the KV cache starts at that many positions and grows in
    256-position chunks up to kv_capacity."""
    from . import GpuLlamaModel

    m = GpuLlamaModel(ctx, cfg, kv_capacity, kv_initial=kv_initial)
    if stream_cache_bytes is not None:
        m.enable_streaming(stream_cache_bytes)
        m.set_cache_policy(cache_policy)
        m.set_persistent_policy(persistent_policy)
    for s in specs:
        m.synth_tensor(s.name, s.ggml_type, s.ne0, s.ne1, s.seed, s.scale_mul, s.constant)
    return m


def write_model_file(ctx, specs: list[TensorSpec], path: str, chunk_bytes: int = 256 << 20) -> dict:
    """Writes the block tensors (blk.*) of `specs` to a file laid out as a
    GGUF tensor-data section (each tensor 32-byte aligned, in spec order, so
    a layer's tensors are contiguous), generating each payload on the device
    (rf_synth_blocks, the bytes rf_model_synth_tensor installs) and copying
    it back in chunks.  Returns {name: (offset, nbytes)}."""
    import numpy as np

    geo = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
    spans = {}
    off = 0
    buf = ctx.empty((chunk_bytes,), np.uint8, charge="synthetic:file_chunk")
    try:
        with open(path, "wb") as f:
            for s in specs:
                if not s.name.startswith("blk."):
                    continue
                off = (off + 31) // 32 * 32
                f.seek(off)
                qk, bs = geo[s.ggml_type]
                nblk = s.ne0 // qk * s.ne1
                spans[s.name] = (off, nblk * bs)
                if s.ggml_type == F32 and s.constant == s.constant:  # a constant fill (norm weights)
                    f.write(np.full(nblk, s.constant, np.float32).tobytes())
                else:
                    per = chunk_bytes // bs
                    for b0 in range(0, nblk, per):
                        n = min(per, nblk - b0)
                        ctx.synth_blocks(s.ggml_type, s.seed, b0, n, s.scale_mul, buf)
                        f.write(buf.numpy()[: n * bs].tobytes())
                off += nblk * bs
    finally:
        buf.free()
    return spans


def build_file_model(ctx, cfg: dict, specs: list[TensorSpec], path: str, spans: dict, kv_capacity: int,
                     stream_cache_bytes: int, cache_policy: int = 1, kv_initial: int | None = None,
                     persistent_policy: int = 0, staging_bytes: int = 64 << 20, threads: int = 8):
    """A streaming GpuLlamaModel whose block tensors are read from the model
    file written by write_model_file (a FileSource: the library's own
    multi-threaded pread reader, `staging_bytes` per pinned staging buffer)
    each time their layer is loaded; the embedding, output norm and output
    projection are generated on the device as in build_device_model."""
    from . import FileSource, GpuLlamaModel

    m = GpuLlamaModel(ctx, cfg, kv_capacity, kv_initial=kv_initial)
    m.enable_streaming(stream_cache_bytes)
    m.set_cache_policy(cache_policy)
    m.set_persistent_policy(persistent_policy)
    src = FileSource(path, threads)
    m.set_reader(src, staging_bytes)
    for s in specs:
        if s.name in spans:
            o, nb = spans[s.name]
            m.set_tensor_source(s.name, s.ggml_type, s.ne0, s.ne1, o, nb)
        else:
            m.synth_tensor(s.name, s.ggml_type, s.ne0, s.ne1, s.seed, s.scale_mul, s.constant)
    return m
