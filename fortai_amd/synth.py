"""Seeded synthetic Qwen3.5-shaped GGUF models and Q8_0 inputs.

There is no network and no real checkpoint, so every model used by the tests
and the bench is generated here from a seed, bit-identically on any machine
with this image.  Tensor names and metadata keys are the ones the reference
binds (``src/models/qwen35/fortai_qwen35_cpu.f90:175-212,1043-1064``); the
tied fp16 ``token_embd.weight`` with no ``output.weight`` exercises the tie at
``:212``.

Distributions (BASELINE configs 1 and 4):
- Q8_0 matrices: quants i.i.d. uniform integers in [-127, 127]; one fp16
  scale per 32-block with |scale| log-uniform in [1e-3, 1e-1] and a random
  sign (fp16 rounding is round-to-nearest-even, numpy's ``astype``).
- tied fp16 embedding ~ N(0, 0.02); RMSNorm weights 1 + N(0, 0.05);
  ssm_a = -exp(N(0, 0.5)) (so the decay is < 1); ssm_dt.bias ~ N(0, 1);
  conv1d weights ~ N(0, 0.1).
"""

from __future__ import annotations

import zlib
from dataclasses import dataclass, asdict
from typing import Dict, Iterator, Tuple

import numpy as np

from . import gguf


@dataclass(frozen=True)
class Qwen35Config:
    name: str
    hidden: int
    layers: int
    ffn: int
    heads: int
    kv_heads: int
    head_size: int
    value_size: int
    rope_dim: int
    gdn_key_heads: int
    gdn_value_heads: int
    gdn_state: int
    gdn_inner: int
    conv_kernel: int
    vocab: int
    interval: int = 4
    eps: float = 1.0e-6
    rope_base: float = 1.0e7
    embedding_q8: bool = False  # tied token_embd as Q8_0 (as llama.cpp Q8_0 exports) instead of F16
    # factor on the attn_v block scales: large enough and the value projection
    # leaves the fp16 range, so the KV cache holds exponent-31 halves
    value_gain: float = 1.0

    @property
    def conv_size(self) -> int:
        # fortai_qwen35_cpu.f90:237-238
        return 2 * self.gdn_state * self.gdn_key_heads + self.gdn_inner

    @property
    def gdn_head(self) -> int:
        return self.gdn_inner // self.gdn_value_heads

    def recurrent(self, layer: int) -> bool:
        """Layer ``layer`` (0-based) is a GDN layer iff mod(layer+1, interval) != 0
        (fortai_qwen35_cpu.f90:247)."""
        return (layer + 1) % self.interval != 0


CONFIGS: Dict[str, Qwen35Config] = {
    # BASELINE config 4 (Qwen3.5-0.8B shape).
    "qwen35-0.8b": Qwen35Config("qwen35-0.8b", hidden=1024, layers=24, ffn=3584, heads=8,
                                kv_heads=2, head_size=256, value_size=256, rope_dim=64,
                                gdn_key_heads=16, gdn_value_heads=16, gdn_state=128,
                                gdn_inner=2048, conv_kernel=4, vocab=248320),
    # A small model with the same structure for fast CPU-oracle parity:
    # GDN value heads > key heads (ratio 2) exercises the grouped mapping.
    "qwen35-tiny": Qwen35Config("qwen35-tiny", hidden=256, layers=4, ffn=512, heads=4,
                                kv_heads=2, head_size=64, value_size=64, rope_dim=16,
                                gdn_key_heads=2, gdn_value_heads=4, gdn_state=64,
                                gdn_inner=256, conv_kernel=4, vocab=4096),
    # The tiny model with a Q8_0 tied embedding / LM head: the tensor types the
    # reference's device pipeline requires (fortai_qwen35_cpu.f90:407-410).
    "qwen35-tiny-q8emb": Qwen35Config("qwen35-tiny-q8emb", hidden=256, layers=4, ffn=512, heads=4,
                                      kv_heads=2, head_size=64, value_size=64, rope_dim=16,
                                      gdn_key_heads=2, gdn_value_heads=4, gdn_state=64,
                                      gdn_inner=256, conv_kernel=4, vocab=4096, embedding_q8=True),
    # The tiny model with value projections of |v| up to ~2e5: fp16 KV appends
    # of exponent-31 halves (read back as +-huge by gguf_fp16_to_real), the
    # attention kernels' flagged path.
    "qwen35-tiny-hugev": Qwen35Config("qwen35-tiny-hugev", hidden=256, layers=4, ffn=512, heads=4,
                                      kv_heads=2, head_size=64, value_size=64, rope_dim=16,
                                      gdn_key_heads=2, gdn_value_heads=4, gdn_state=64,
                                      gdn_inner=256, conv_kernel=4, vocab=4096, value_gain=1000.0),
    # Mid-size: every 0.8B layer shape except the vocabulary and depth.
    "qwen35-0.8b-short": Qwen35Config("qwen35-0.8b-short", hidden=1024, layers=4, ffn=3584,
                                      heads=8, kv_heads=2, head_size=256, value_size=256,
                                      rope_dim=64, gdn_key_heads=16, gdn_value_heads=16,
                                      gdn_state=128, gdn_inner=2048, conv_kernel=4,
                                      vocab=16384),
    # The mid-size model with a Q8_0 tied embedding / LM head, so that the
    # reference's own device pipeline runs at the 0.8B layer shapes.
    "qwen35-0.8b-short-q8emb": Qwen35Config("qwen35-0.8b-short-q8emb", hidden=1024, layers=4, ffn=3584,
                                            heads=8, kv_heads=2, head_size=256, value_size=256,
                                            rope_dim=64, gdn_key_heads=16, gdn_value_heads=16,
                                            gdn_state=128, gdn_inner=2048, conv_kernel=4,
                                            vocab=16384, embedding_q8=True),
    # BASELINE config 5 (Qwen3.5-4B shape): hidden 2560, 32 layers (24 GDN /
    # 8 attention), FFN 9216, 16 q / 4 kv heads of 256.  BASELINE leaves the
    # GDN heads open; 16 key / 32 value heads of 128 (value_heads % key_heads
    # == 0, fortai_qwen35_cpu.f90:231-235) give conv channels 8192, inner 4096.
    "qwen35-4b": Qwen35Config("qwen35-4b", hidden=2560, layers=32, ffn=9216, heads=16, kv_heads=4,
                              head_size=256, value_size=256, rope_dim=64, gdn_key_heads=16,
                              gdn_value_heads=32, gdn_state=128, gdn_inner=4096, conv_kernel=4,
                              vocab=248320),
    # Every 4B layer shape with 4 layers and a small vocabulary (fast parity).
    "qwen35-4b-short": Qwen35Config("qwen35-4b-short", hidden=2560, layers=4, ffn=9216, heads=16,
                                    kv_heads=4, head_size=256, value_size=256, rope_dim=64,
                                    gdn_key_heads=16, gdn_value_heads=32, gdn_state=128,
                                    gdn_inner=4096, conv_kernel=4, vocab=16384),
}


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed & 0xFFFFFFFF, zlib.crc32(name.encode())])


def q8_blocks(rng: np.random.Generator, rows: int, width: int) -> np.ndarray:
    """GGUF Q8_0 bytes [rows][width/32][34] with the BASELINE config-1 distribution."""
    blocks = width // gguf.Q8_BLOCK
    out = np.empty((rows, blocks, gguf.Q8_BLOCK_BYTES), dtype=np.uint8)
    chunk = max(1, (1 << 22) // max(blocks, 1))
    for start in range(0, rows, chunk):
        stop = min(rows, start + chunk)
        n = stop - start
        magnitude = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), size=(n, blocks)))
        sign = np.where(rng.integers(0, 2, size=(n, blocks)) == 0, -1.0, 1.0)
        scale = (magnitude * sign).astype(np.float16)
        quants = rng.integers(-127, 128, size=(n, blocks, gguf.Q8_BLOCK), dtype=np.int8)
        out[start:stop, :, 0:2] = scale.view(np.uint8).reshape(n, blocks, 2)
        out[start:stop, :, 2:] = quants.view(np.uint8)
    return out


def _normal(rng: np.random.Generator, n: int, std: float, dtype) -> np.ndarray:
    out = np.empty(n, dtype=dtype)
    chunk = 1 << 24
    for start in range(0, n, chunk):
        stop = min(n, start + chunk)
        out[start:stop] = (rng.standard_normal(stop - start, dtype=np.float32) * np.float32(std)).astype(dtype)
    return out


def tensor_specs(cfg: Qwen35Config) -> Iterator[Tuple[str, Tuple[int, ...], int]]:
    f32, f16, q8 = gguf.GGML_TYPE_F32, gguf.GGML_TYPE_F16, gguf.GGML_TYPE_Q8_0
    h = cfg.hidden
    yield "token_embd.weight", (h, cfg.vocab), (q8 if cfg.embedding_q8 else f16)
    yield "output_norm.weight", (h,), f32
    for i in range(cfg.layers):
        p = f"blk.{i}."
        yield p + "attn_norm.weight", (h,), f32
        yield p + "post_attention_norm.weight", (h,), f32
        yield p + "ffn_gate.weight", (h, cfg.ffn), q8
        yield p + "ffn_up.weight", (h, cfg.ffn), q8
        yield p + "ffn_down.weight", (cfg.ffn, h), q8
        if cfg.recurrent(i):
            yield p + "attn_qkv.weight", (h, cfg.conv_size), q8
            yield p + "attn_gate.weight", (h, cfg.gdn_inner), q8
            yield p + "ssm_a", (cfg.gdn_value_heads,), f32
            yield p + "ssm_alpha.weight", (h, cfg.gdn_value_heads), q8
            yield p + "ssm_beta.weight", (h, cfg.gdn_value_heads), q8
            yield p + "ssm_conv1d.weight", (cfg.conv_kernel, cfg.conv_size), f32
            yield p + "ssm_dt.bias", (cfg.gdn_value_heads,), f32
            yield p + "ssm_norm.weight", (cfg.gdn_head,), f32
            yield p + "ssm_out.weight", (cfg.gdn_inner, h), q8
        else:
            yield p + "attn_q.weight", (h, 2 * cfg.heads * cfg.head_size), q8
            yield p + "attn_k.weight", (h, cfg.kv_heads * cfg.head_size), q8
            yield p + "attn_v.weight", (h, cfg.kv_heads * cfg.value_size), q8
            yield p + "attn_output.weight", (cfg.heads * cfg.value_size, h), q8
            yield p + "attn_q_norm.weight", (cfg.head_size,), f32
            yield p + "attn_k_norm.weight", (cfg.head_size,), f32


def tensor_payload(cfg: Qwen35Config, seed: int, name: str, shape, ggml_type) -> np.ndarray:
    rng = _rng(seed, name)
    n = int(np.prod(shape))
    if ggml_type == gguf.GGML_TYPE_Q8_0:
        blocks = q8_blocks(rng, int(np.prod(shape[1:])), shape[0])
        if cfg.value_gain != 1.0 and name.endswith("attn_v.weight"):
            sc = blocks[..., 0:2].copy().view(np.float16).astype(np.float32) * np.float32(cfg.value_gain)
            blocks[..., 0:2] = np.clip(sc, -60000.0, 60000.0).astype(np.float16).view(np.uint8)
        return blocks
    if ggml_type == gguf.GGML_TYPE_F16:
        return _normal(rng, n, 0.02, np.float16)
    base = name.split(".", 2)[-1]
    if base == "ssm_a":
        return (-np.exp(rng.normal(0.0, 0.5, size=n))).astype(np.float32)
    if base == "ssm_dt.bias":
        return rng.standard_normal(n).astype(np.float32)
    if base == "ssm_conv1d.weight":
        return (rng.standard_normal(n) * 0.1).astype(np.float32)
    # RMSNorm-style weights
    return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)


def write_model(path: str, cfg: Qwen35Config, seed: int = 0x51E5) -> None:
    """Write a complete synthetic Qwen3.5 GGUF v3 file (keys as the reference reads them)."""
    w = gguf.Writer(path)
    U32, F32 = gguf.GGUF_UINT32, gguf.GGUF_FLOAT32
    w.add_meta("general.architecture", gguf.GGUF_STRING, "qwen35")
    w.add_meta("general.name", gguf.GGUF_STRING, f"fortai-synthetic-{cfg.name}-seed{seed}")
    meta = {
        "qwen35.embedding_length": cfg.hidden, "qwen35.vocab_size": cfg.vocab,
        "qwen35.block_count": cfg.layers, "qwen35.feed_forward_length": cfg.ffn,
        "qwen35.attention.head_count": cfg.heads, "qwen35.attention.head_count_kv": cfg.kv_heads,
        "qwen35.attention.key_length": cfg.head_size, "qwen35.attention.value_length": cfg.value_size,
        "qwen35.rope.dimension_count": cfg.rope_dim, "qwen35.ssm.conv_kernel": cfg.conv_kernel,
        "qwen35.ssm.state_size": cfg.gdn_state, "qwen35.ssm.group_count": cfg.gdn_key_heads,
        "qwen35.ssm.time_step_rank": cfg.gdn_value_heads, "qwen35.ssm.inner_size": cfg.gdn_inner,
        "qwen35.full_attention_interval": cfg.interval,
        "tokenizer.ggml.bos_token_id": 0, "tokenizer.ggml.eos_token_id": 1,
    }
    for key, value in meta.items():
        w.add_meta(key, U32, value)
    w.add_meta("qwen35.attention.layer_norm_rms_epsilon", F32, cfg.eps)
    w.add_meta("qwen35.rope.freq_base", F32, cfg.rope_base)
    specs = list(tensor_specs(cfg))
    shapes = {}
    for name, shape, ggml_type in specs:
        w.add_tensor(name, shape, ggml_type)
        shapes[name] = (shape, ggml_type)
    w.write(lambda name: tensor_payload(cfg, seed, name, *shapes[name]))


def config_dict(cfg: Qwen35Config) -> dict:
    return asdict(cfg)


def matvec_inputs(rows: int = 3584, width: int = 1024, seed: int = 0x6F727461):
    """GGUF Q8_0 W [rows x width] and x ~ N(0,1) f32[width]."""
    rng = np.random.default_rng(seed)
    w = q8_blocks(rng, rows, width)
    x = rng.standard_normal(width).astype(np.float32)
    return w, x
