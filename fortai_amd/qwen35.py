"""Host driver of the Qwen3.5 decode step on the gfx950 backend.

Mirrors the reference model's device path (src/models/qwen35/fortai_qwen35_cpu.f90):
config from GGUF metadata (:175-238), layer pattern mod(i, interval) != 0 ->
recurrent (:247), resident upload of every 2-D Q8_0 tensor and per-layer
device objects (enable_cuda, :287-384), then ``forward(token, position)``
(:591-711) and the greedy runner loop (app/fortai_cpu_run.f90:50-64).

Two execution modes over the same device objects:
* ``forward`` / ``generate``: the fused decoder (one HIP graph per token,
  greedy argmax on device) -- the production path;
* ``forward_ops``: the reference ABI call sequence per layer (copy, rms_norm,
  run_device, add, copy, rms_norm, ffn_device, add; :713-799), used to check
  the drop-in entry points end to end.
The tied fp16 embedding/LM head, which the reference CUDA pipeline cannot keep
device-resident (:410-413), is resident here.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import backend as B
from . import gguf


@dataclass
class Qwen35Dims:
    hidden: int
    vocab: int
    layers: int
    ffn: int
    heads: int
    kv_heads: int
    head_size: int
    value_size: int
    rope_dim: int
    conv_kernel: int
    state_size: int
    key_heads: int
    value_heads: int
    inner: int
    interval: int
    eps: float
    rope_base: float

    @property
    def gdn_head(self) -> int:
        return self.inner // self.value_heads

    @property
    def conv_size(self) -> int:
        return 2 * self.state_size * self.key_heads + self.inner


def read_dims(f: gguf.GGUFFile) -> Qwen35Dims:
    """fortai_qwen35_cpu.f90:175-238"""
    d = Qwen35Dims(
        hidden=f.meta_int("qwen35.embedding_length"), vocab=f.meta_int("qwen35.vocab_size"),
        layers=f.meta_int("qwen35.block_count"), ffn=f.meta_int("qwen35.feed_forward_length"),
        heads=f.meta_int("qwen35.attention.head_count"), kv_heads=f.meta_int("qwen35.attention.head_count_kv"),
        head_size=f.meta_int("qwen35.attention.key_length"), value_size=f.meta_int("qwen35.attention.value_length"),
        rope_dim=f.meta_int("qwen35.rope.dimension_count"), conv_kernel=f.meta_int("qwen35.ssm.conv_kernel"),
        state_size=f.meta_int("qwen35.ssm.state_size"), key_heads=f.meta_int("qwen35.ssm.group_count"),
        value_heads=f.meta_int("qwen35.ssm.time_step_rank"), inner=f.meta_int("qwen35.ssm.inner_size"),
        interval=f.meta_int("qwen35.full_attention_interval", 4),
        eps=f.meta_real("qwen35.attention.layer_norm_rms_epsilon", 1.0e-6),
        rope_base=f.meta_real("qwen35.rope.freq_base", 1.0e7))
    emb = f.tensor("token_embd.weight")
    if emb is not None and len(emb.shape) == 2:
        d.hidden, d.vocab = emb.shape[0], emb.shape[1]
    if min(d.hidden, d.vocab, d.layers, d.ffn, d.heads, d.kv_heads, d.head_size, d.state_size, d.inner,
           d.interval) <= 0:
        raise ValueError("GGUF does not contain a complete Qwen3.5 config")
    if d.inner % d.value_heads or d.value_heads % d.key_heads or d.heads % d.kv_heads:
        raise ValueError("Qwen3.5 head groups are not divisible")
    return d


class Qwen35Hip:
    def __init__(self, path: str, max_context: int = 256, device: int = 0, fused: bool = True, batch: int = 0,
                 pack_cache: Optional[str] = None, direct: bool = False, exact_max: Optional[int] = None):
        """pack_cache: root of a repacked-weight cache (fortai_amd.pack_cache);
        the Q8_0 matrices are uploaded from it when it holds this GGUF's pack,
        and the pack is written after a repacking upload otherwise.
        direct: the decoders enqueue their kernels every step instead of
        replaying a captured graph (same results; for kernel tracing).
        exact_max: the attention layers' exact-softmax limit (default 8192)."""
        self.file = gguf.read(path)
        self.d = d = read_dims(self.file)
        self.max_context = max_context
        self.ctx = B.Context(device)
        self.q8: Dict[str, B.Q8Weights] = {}
        packed = None
        self.pack_path = None
        self.loaded_from_pack = False
        if pack_cache:
            from . import pack_cache as pc
            digest = pc.gguf_digest(path)
            self.pack_path = pc.cache_path(pack_cache, pc.model_key(path))
            packed = pc.read(self.pack_path, digest)
        for t in self.file.tensors:
            if t.ggml_type == gguf.GGML_TYPE_Q8_0 and len(t.shape) == 2:
                rec = packed.get(t.name) if packed else None
                if rec is not None and rec[0] == t.rows and rec[1] == t.width:
                    self.q8[t.name] = B.Q8Weights.from_packed(self.ctx, rec[2], t.rows, t.width)
                else:
                    self.q8[t.name] = B.Q8Weights(self.ctx, t.data, t.rows, t.width)
        self.loaded_from_pack = bool(packed) and len(packed) == len(self.q8)
        if pack_cache and not self.loaded_from_pack:
            pc.write(self.pack_path, digest, {n: (w.rows, w.width, w.pack()) for n, w in self.q8.items()})
        emb = self.file.tensor("token_embd.weight")
        out = self.file.tensor("output.weight") or emb
        self.f16: Dict[str, B.F16Weights] = {}
        for t in {emb.name: emb, out.name: out}.values():
            if t.ggml_type == gguf.GGML_TYPE_F16:
                self.f16[t.name] = B.F16Weights(self.ctx, t.data, t.rows, t.width)
        self.embedding = self.f16.get(emb.name) or self.q8.get(emb.name)
        self.output = self.f16.get(out.name) or self.q8.get(out.name)
        if self.embedding is None or self.output is None:
            raise ValueError("token embedding / output must be F16 or Q8_0")
        self.recurrent: List[Optional[B.Recurrent]] = []
        self.attention: List[Optional[B.Attention]] = []
        self.norms: List[Dict[str, np.ndarray]] = []
        for i in range(d.layers):
            p = f"blk.{i}."
            T = lambda n: self.file.tensor(p + n)
            Q = lambda n: self.q8[p + n]
            self.norms.append({"attn": T("attn_norm.weight").as_f32(), "post": T("post_attention_norm.weight").as_f32()})
            if (i + 1) % d.interval != 0:
                self.recurrent.append(B.Recurrent(
                    self.ctx, Q("attn_qkv.weight"), Q("attn_gate.weight"), Q("ssm_alpha.weight"),
                    Q("ssm_beta.weight"), Q("ssm_out.weight"), T("ssm_conv1d.weight").as_f32(), d.conv_size,
                    d.conv_kernel, T("ssm_a").as_f32(), T("ssm_dt.bias").as_f32(), T("ssm_norm.weight").as_f32(),
                    d.state_size, d.key_heads, d.value_heads, d.gdn_head, d.inner, d.eps))
                self.attention.append(None)
            else:
                self.recurrent.append(None)
                self.attention.append(B.Attention(
                    self.ctx, Q("attn_q.weight"), Q("attn_k.weight"), Q("attn_v.weight"), Q("attn_output.weight"),
                    T("attn_q_norm.weight").as_f32(), T("attn_k_norm.weight").as_f32(), d.heads, d.kv_heads,
                    d.head_size, d.value_size, max_context, d.rope_dim, d.rope_base, d.eps))
        if exact_max is not None:
            for a in self.attention:
                if a is not None:
                    a.set_exact_max(exact_max)
        self.output_norm = self.file.tensor("output_norm.weight").as_f32()
        self.decoder: Optional[B.Decoder] = None
        if fused:
            self.decoder = B.Decoder(
                self.ctx, self.recurrent, self.attention,
                [self.q8[f"blk.{i}.ffn_gate.weight"] for i in range(d.layers)],
                [self.q8[f"blk.{i}.ffn_up.weight"] for i in range(d.layers)],
                [self.q8[f"blk.{i}.ffn_down.weight"] for i in range(d.layers)],
                [n["attn"] for n in self.norms], [n["post"] for n in self.norms], self.output_norm, d.hidden,
                self.embedding, self.output, max_context, d.eps, d.vocab)
            if direct:
                self.decoder.set_mode(direct=True)
        self.batch: Optional[B.BatchDecoder] = None
        if batch:
            self.batch = B.BatchDecoder(
                self.ctx, batch, self.recurrent, self.attention,
                [self.q8[f"blk.{i}.ffn_gate.weight"] for i in range(d.layers)],
                [self.q8[f"blk.{i}.ffn_up.weight"] for i in range(d.layers)],
                [self.q8[f"blk.{i}.ffn_down.weight"] for i in range(d.layers)],
                [n["attn"] for n in self.norms], [n["post"] for n in self.norms], self.output_norm, d.hidden,
                self.embedding, self.output, max_context, d.eps, d.vocab)
            if direct:
                self.batch.set_mode(direct=True)
        self._ops = None

    # ---------------------------------------------------------------- fused
    def reset(self) -> None:
        if self.decoder:
            self.decoder.reset()
        else:
            for layer in self.recurrent + self.attention:
                if layer is not None:
                    layer.reset()

    def forward(self, token: int, position: int) -> np.ndarray:
        self.decoder.forward(token, position)
        return self.decoder.logits

    def generate(self, token: int, steps: int, start: int = 0) -> np.ndarray:
        return self.decoder.generate(token, start, steps)

    # ------------------------------------------------------ reference ABI ops
    def _op_buffers(self):
        if self._ops is None:
            d = self.d
            ctx = self.ctx
            hb = d.hidden * 4
            self._ops = {
                "x": ctx.alloc(hb), "residual": ctx.alloc(hb), "normalized": ctx.alloc(hb), "hidden": ctx.alloc(hb),
                "logits": ctx.alloc(d.vocab * 4), "token": ctx.alloc(8),
                "onorm": ctx.upload_array(self.output_norm),
                "attn": [ctx.upload_array(n["attn"]) for n in self.norms],
                "post": [ctx.upload_array(n["post"]) for n in self.norms],
            }
        return self._ops

    def forward_ops(self, token: int, position: int) -> np.ndarray:
        """One token through the per-op reference ABI (fortai_qwen35_cpu.f90:612-706)."""
        d, ctx, b = self.d, self.ctx, self._op_buffers()
        H = d.hidden
        if isinstance(self.embedding, B.F16Weights):
            ctx.call("fortai_hip_qwen35_embedding_f16_device", ctx.h, self.embedding.h, token, b["x"].ptr, H)
        else:
            ctx.call("fortai_hip_qwen35_embedding_device", ctx.h, self.embedding.h, token, b["x"].ptr, H)
        ctx.set_position(position)
        for i in range(d.layers):
            ctx.call("fortai_hip_qwen35_copy_device", ctx.h, b["x"].ptr, b["residual"].ptr, H * 4)
            ctx.call("fortai_hip_qwen35_rms_norm_device", ctx.h, b["x"].ptr, b["attn"][i].ptr, b["normalized"].ptr,
                     H, d.eps)
            if self.recurrent[i] is not None:
                ctx.call("fortai_hip_qwen35_recurrent_run_device", self.recurrent[i].h, b["normalized"].ptr, H,
                         b["hidden"].ptr, H)
            else:
                ctx.call("fortai_hip_qwen35_attention_run_device", self.attention[i].h, b["normalized"].ptr, H,
                         position, b["hidden"].ptr, H)
            ctx.call("fortai_hip_qwen35_add_device", ctx.h, b["hidden"].ptr, b["residual"].ptr, b["x"].ptr, H)
            ctx.call("fortai_hip_qwen35_copy_device", ctx.h, b["x"].ptr, b["residual"].ptr, H * 4)
            ctx.call("fortai_hip_qwen35_rms_norm_device", ctx.h, b["x"].ptr, b["post"][i].ptr, b["normalized"].ptr,
                     H, d.eps)
            p = f"blk.{i}."
            ctx.call("fortai_hip_q8_ffn_device", ctx.h, self.q8[p + "ffn_gate.weight"].h,
                     self.q8[p + "ffn_up.weight"].h, self.q8[p + "ffn_down.weight"].h, b["normalized"].ptr, H,
                     b["hidden"].ptr, H)
            ctx.call("fortai_hip_qwen35_add_device", ctx.h, b["hidden"].ptr, b["residual"].ptr, b["x"].ptr, H)
        ctx.call("fortai_hip_qwen35_rms_norm_device", ctx.h, b["x"].ptr, b["onorm"].ptr, b["normalized"].ptr, H,
                 d.eps)
        if isinstance(self.output, B.F16Weights):
            ctx.call("fortai_hip_f16_matvec_device", ctx.h, self.output.h, b["normalized"].ptr, H,
                     b["logits"].ptr, d.vocab, b["token"].ptr)
        else:
            ctx.call("fortai_hip_q8_matvec_device_f32", ctx.h, self.output.h, b["normalized"].ptr, H,
                     b["logits"].ptr, d.vocab)
        return b["logits"].download(np.float32, d.vocab)

    def close(self) -> None:
        if self.batch:
            self.batch.free()
        if self.decoder:
            self.decoder.free()
        if self._ops:
            for v in self._ops.values():
                for buf in (v if isinstance(v, list) else [v]):
                    buf.free()
        for layer in self.recurrent:
            if layer:
                layer.free()
        for layer in self.attention:
            if layer:
                layer.free()
        for w in list(self.q8.values()) + list(self.f16.values()):
            w.free()
        self.ctx.close()
