"""ctypes mirror of the gfx950 C ABI (include/fortai_hip_backend.h).

Python counterpart of the reference's iso_c_binding wrapper
(src/backend/cuda/fortai_backend_cuda.f90): opaque handles with create /
destroy, and every nonzero return code raised as ``BackendError`` with the
context's last error message (the wrapper maps them to status_t,
fortai_backend_cuda.f90:418-431).  There is no CPU fallback: if
``libfortai_hip.so`` is missing or no GPU is visible, creating a context raises.
"""

from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

# the in-tree build; FORTAI_HIP_LIBRARY names another build of the same library
LIB_PATH = os.environ.get("FORTAI_HIP_LIBRARY") or \
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libfortai_hip.so")

OK, INVALID, RUNTIME_ERROR = 0, 1, 2

_vp, _i, _i64, _sz, _f = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float
_fp, _i64p, _u16p = C.POINTER(C.c_float), C.POINTER(C.c_int64), C.POINTER(C.c_uint16)
_vpp = C.POINTER(C.c_void_p)

# name -> argtypes (all return int unless listed in _RESTYPE)
_SIGNATURES = {
    "fortai_hip_q8_context_create": [_i, _vpp],
    "fortai_hip_q8_context_destroy": [_vp],
    "fortai_hip_q8_context_set_position": [_vp, _i],
    "fortai_hip_q8_context_capture_begin": [_vp],
    "fortai_hip_q8_context_capture_end": [_vp],
    "fortai_hip_q8_context_graph_launch": [_vp],
    "fortai_hip_q8_context_synchronize": [_vp],
    "fortai_hip_q8_context_scratch_bytes": [_vp, C.POINTER(C.c_size_t)],
    "fortai_hip_q8_context_timer_start": [_vp],
    "fortai_hip_q8_context_timer_stop": [_vp, _fp],
    "fortai_hip_q8_weights_upload": [_vp, _vp, _sz, _i, _i, _vpp],
    "fortai_hip_q8_weights_destroy": [_vp],
    "fortai_hip_q8_device_buffer_create": [_vp, _sz, _vpp],
    "fortai_hip_q8_device_buffer_destroy": [_vp, _vp],
    "fortai_hip_q8_device_buffer_upload": [_vp, _vp, _vp, _sz],
    "fortai_hip_q8_device_buffer_upload_ptr": [_vp, _vp, _vp, _sz],
    "fortai_hip_q8_device_buffer_download": [_vp, _vp, _vp, _sz],
    "fortai_hip_q8_matvec_resident": [_vp, _vp, _vp, _vp, _fp],
    "fortai_hip_q8_matvec_device_f32": [_vp, _vp, _vp, _sz, _vp, _sz],
    "fortai_hip_qwen35_embedding_device": [_vp, _vp, _i64, _vp, _sz],
    "fortai_hip_qwen35_copy_device": [_vp, _vp, _vp, _sz],
    "fortai_hip_qwen35_add_device": [_vp, _vp, _vp, _vp, _sz],
    "fortai_hip_qwen35_rms_norm_device": [_vp, _vp, _vp, _vp, _sz, _f],
    "fortai_hip_q8_matvec_host": [_vp, _vp, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_q8_matvec_host_pair": [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_q8_matvec_host_triplet": [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_q8_matvec_host_triplet_contiguous": [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_q8_ffn_host": [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_q8_ffn_device": [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz],
    "fortai_hip_qwen35_recurrent_create": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _vp, _sz, _vp, _sz,
                                           _vp, _sz, _i, _i, _i, _i, _i, _f, _vpp],
    "fortai_hip_qwen35_recurrent_destroy": [_vp],
    "fortai_hip_qwen35_recurrent_reset": [_vp],
    "fortai_hip_qwen35_recurrent_run": [_vp, _vp, _sz, _vp, _sz, _fp],
    "fortai_hip_qwen35_recurrent_run_device": [_vp, _vp, _sz, _vp, _sz],
    "fortai_hip_qwen35_attention_create": [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _i, _i, _i, _i, _i, _i,
                                           _f, _f, _vpp],
    "fortai_hip_qwen35_attention_destroy": [_vp],
    "fortai_hip_qwen35_attention_reset": [_vp],
    "fortai_hip_qwen35_attention_run_device": [_vp, _vp, _sz, _i, _vp, _sz],
    "fortai_hip_q8_last_error": [_vp],
    "fortai_hip_f16_weights_upload": [_vp, _vp, _sz, _i, _i, _vpp],
    "fortai_hip_f16_weights_destroy": [_vp],
    "fortai_hip_f16_matvec_device": [_vp, _vp, _vp, _sz, _vp, _sz, _vp],
    "fortai_hip_qwen35_embedding_f16_device": [_vp, _vp, _i64, _vp, _sz],
    "fortai_hip_argmax_device": [_vp, _vp, _sz, _vp],
    "fortai_hip_q8_quantize_device": [_vp, _vp, _sz, _vp, _vp],
    "fortai_hip_q8_block_dots_device": [_vp, _vp, _vp, _vp],
    "fortai_hip_q8_batch_matvec_noalloc": [_vp, _vp, _vp, _i, _vp],
    "fortai_hip_q8_batch_matvec_device": [_vp, _vp, _vp, _i, _vp, _fp],
    "fortai_hip_q8_pack_bytes": [_i, _i],
    "fortai_hip_q8_weights_pack": [_vp, _vp, _sz],
    "fortai_hip_q8_weights_upload_packed": [_vp, _vp, _sz, _i, _i, _vpp],
    "fortai_hip_q8_tokens_bytes": [_i, _i],
    "fortai_hip_q8_quantize_tokens_device": [_vp, _vp, _i, _i, _vp],
    "fortai_hip_q8_mmq_device": [_vp, _vp, _vp, _i, _vp, _vp, _fp],
    "fortai_hip_q8_mmq_exact_device": [_vp, _vp, _vp, _i, _vp, _vp, _fp],
    "fortai_hip_q8_mmq_block_dots": [_vp, _vp, _vp, _i, _vp],
    "fortai_hip_qwen35_recurrent_core_steps_device": [_vp, _vp, _vp, _vp, _i, _vp],
    "fortai_hip_qwen35_recurrent_core_device": [_vp, _vp, _vp, _vp, _vp],
    "fortai_hip_qwen35_recurrent_state_download": [_vp, _vp, _sz, _vp, _sz],
    "fortai_hip_qwen35_recurrent_state_upload": [_vp, _vp, _sz, _vp, _sz],
    "fortai_hip_qwen35_attention_core_device": [_vp, _vp, _vp, _vp, _vp],
    "fortai_hip_qwen35_attention_prefill_core_device": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "fortai_hip_qwen35_attention_cache_download": [_vp, _vp, _vp, _i],
    "fortai_hip_qwen35_attention_cache_upload": [_vp, _vp, _vp, _i],
    "fortai_hip_qwen35_decoder_create": [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                                         _i, _f, _vpp],
    "fortai_hip_qwen35_decoder_destroy": [_vp],
    "fortai_hip_qwen35_decoder_reset": [_vp],
    "fortai_hip_qwen35_decoder_forward": [_vp, _i64, _i, _vp, _vp],
    "fortai_hip_qwen35_decoder_generate": [_vp, _i64, _i, _i, _vp],
    "fortai_hip_qwen35_decoder_replay": [_vp, _i],
    "fortai_hip_qwen35_decoder_logits": [_vp, _vpp],
    "fortai_hip_qwen35_decoder_trace": [_vp, _i, _i, _vp],
    "fortai_hip_qwen35_decoder_status": [_vp],
    "fortai_hip_qwen35_decoder_plan": [_vp, _vp, _sz, C.POINTER(C.c_size_t)],
    "fortai_hip_qwen35_batch_plan": [_vp, _i, _vp, _sz, C.POINTER(C.c_size_t)],
    "fortai_hip_qwen35_batch_create": [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp,
                                       _vp, _i, _f, _vpp],
    "fortai_hip_qwen35_batch_destroy": [_vp],
    "fortai_hip_qwen35_batch_reset": [_vp],
    "fortai_hip_qwen35_batch_forward": [_vp, _vp, _vp, _vp, _vp],
    "fortai_hip_qwen35_batch_generate": [_vp, _vp, _vp, _i, _vp],
    "fortai_hip_qwen35_batch_replay": [_vp, _i],
    "fortai_hip_qwen35_batch_logits": [_vp, _vpp],
    "fortai_hip_qwen35_batch_prefill": [_vp, _vp, _i, _vp, _vp, _fp],
    "fortai_hip_qwen35_attention_set_exact_max": [_vp, _i],
    "fortai_hip_qwen35_attention_set_test_options": [_vp, _i, _i],
    "fortai_hip_qwen35_decoder_set_mode": [_vp, _i],
    "fortai_hip_qwen35_batch_set_mode": [_vp, _i],
    "fortai_hip_qwen35_batch_set_prefill_mode": [_vp, _i],
}
_RESTYPE = {"fortai_hip_q8_last_error": C.c_char_p, "fortai_hip_q8_tokens_bytes": C.c_size_t,
            "fortai_hip_q8_pack_bytes": C.c_size_t}

_lib: Optional[C.CDLL] = None


# option values of include/fortai_hip_backend.h
DECODER_DIRECT = 1
DECODER_MATVEC_ONLY = 2
DECODER_FAMILIES = {"matvec": 2, "gdn": 4, "attention": 8, "head": 16}
PREFILL_MODES = {"exact": 0, "matvec": 1, "fast": 2}


class BackendError(RuntimeError):
    def __init__(self, code: int, what: str, message: str = ""):
        super().__init__(f"{what} failed with code {code}" + (f": {message}" if message else ""))
        self.code = code


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libfortai_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: run fortai_amd.build.build() (no CPU fallback exists)")
    lib = C.CDLL(path)
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int)
    _lib = lib
    return lib


def exported_symbols() -> Sequence[str]:
    return list(_SIGNATURES)


def _plan(ctx, name: str, *args):
    """Read a recorded plan: [(operation, kernel, batch)] (PlanIR steps)."""
    need = C.c_size_t()
    ctx.call(name, *args, None, 0, C.byref(need))
    buf = C.create_string_buffer(need.value)
    ctx.call(name, *args, buf, need.value, C.byref(need))
    steps = []
    for line in buf.value.decode().splitlines():
        op, kernel, batch = line.split("\t")
        steps.append((op, kernel, int(batch)))
    return steps


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


class Context:
    """A device context: stream, device position/token, scratch (fortai_cuda_q8_context)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = C.c_void_p()
        rc = self.lib.fortai_hip_q8_context_create(device, C.byref(h))
        if rc != OK:
            raise BackendError(rc, "fortai_hip_q8_context_create (is a GPU visible?)")
        self.h = h

    def check(self, rc: int, what: str) -> None:
        if rc != OK:
            msg = self.lib.fortai_hip_q8_last_error(self.h)
            raise BackendError(rc, what, msg.decode() if msg else "")

    def call(self, name: str, *args) -> None:
        self.check(getattr(self.lib, name)(*args), name)

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.fortai_hip_q8_context_destroy(self.h)
            self.h = None

    def set_position(self, position: int) -> None:
        self.call("fortai_hip_q8_context_set_position", self.h, position)

    def scratch_bytes(self) -> int:
        """Bytes of the scratch buffers this context has allocated on demand."""
        n = C.c_size_t()
        self.call("fortai_hip_q8_context_scratch_bytes", self.h, C.byref(n))
        return n.value

    def synchronize(self) -> None:
        self.call("fortai_hip_q8_context_synchronize", self.h)

    def timer_start(self) -> None:
        self.call("fortai_hip_q8_context_timer_start", self.h)

    def timer_stop(self) -> float:
        ms = C.c_float()
        self.call("fortai_hip_q8_context_timer_stop", self.h, C.byref(ms))
        return float(ms.value)

    def capture_begin(self) -> None:
        self.call("fortai_hip_q8_context_capture_begin", self.h)

    def capture_end(self) -> None:
        self.call("fortai_hip_q8_context_capture_end", self.h)

    def graph_launch(self) -> None:
        self.call("fortai_hip_q8_context_graph_launch", self.h)

    # ---- device buffers
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def upload_array(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = DeviceBuffer(self, max(a.nbytes, 1))
        buf.upload(a)
        return buf


class DeviceBuffer:
    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        h = C.c_void_p()
        ctx.call("fortai_hip_q8_device_buffer_create", ctx.h, self.nbytes, C.byref(h))
        self.h = h

    @property
    def ptr(self) -> C.c_void_p:
        return self.h

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        self.ctx.call("fortai_hip_q8_device_buffer_upload", self.ctx.h, self.h, _ptr(a), a.nbytes)

    def download(self, dtype, count: Optional[int] = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        self.ctx.call("fortai_hip_q8_device_buffer_download", self.ctx.h, _ptr(out), self.h, out.nbytes)
        return out

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_q8_device_buffer_destroy(self.ctx.h, self.h)
            self.h = None


class Q8Weights:
    """Resident Q8_0 matrix (GGUF bytes [rows][width/32][34])."""

    def __init__(self, ctx: Context, gguf_bytes: Optional[np.ndarray], rows: int, width: int,
                 packed: Optional[np.ndarray] = None):
        self.ctx, self.rows, self.width = ctx, rows, width
        h = C.c_void_p()
        if packed is not None:
            planes = np.ascontiguousarray(packed).view(np.uint8)
            ctx.call("fortai_hip_q8_weights_upload_packed", ctx.h, _ptr(planes), planes.nbytes, rows, width,
                     C.byref(h))
        else:
            data = np.ascontiguousarray(gguf_bytes).view(np.uint8)
            ctx.call("fortai_hip_q8_weights_upload", ctx.h, _ptr(data), data.nbytes, rows, width, C.byref(h))
        self.h = h

    @classmethod
    def from_packed(cls, ctx: Context, planes: np.ndarray, rows: int, width: int) -> "Q8Weights":
        """A resident matrix from planes written by pack() (no repack)."""
        return cls(ctx, None, rows, width, packed=planes)

    def pack(self) -> np.ndarray:
        """The resident (repacked) planes, for a weight-pack cache."""
        n = self.ctx.lib.fortai_hip_q8_pack_bytes(self.rows, self.width)
        out = np.empty(n, dtype=np.uint8)
        self.ctx.call("fortai_hip_q8_weights_pack", self.h, _ptr(out), n)
        return out

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_q8_weights_destroy(self.h)
            self.h = None


class F16Weights:
    """Resident fp16 matrix (GGUF F16 row-major [rows][width])."""

    def __init__(self, ctx: Context, bits: np.ndarray, rows: int, width: int):
        self.ctx, self.rows, self.width = ctx, rows, width
        data = np.ascontiguousarray(bits).view(np.uint16)
        h = C.c_void_p()
        ctx.call("fortai_hip_f16_weights_upload", ctx.h, _ptr(data), data.nbytes, rows, width, C.byref(h))
        self.h = h

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_f16_weights_destroy(self.h)
            self.h = None


class Recurrent:
    """Qwen3.5 Gated DeltaNet layer (fortai_cuda_qwen35_recurrent)."""

    def __init__(self, ctx: Context, qkv: Q8Weights, gate: Q8Weights, alpha: Q8Weights, beta: Q8Weights,
                 out: Q8Weights, conv_w: np.ndarray, conv_size: int, conv_kernel: int, ssm_a: np.ndarray,
                 ssm_dt: np.ndarray, ssm_norm: np.ndarray, state_size: int, key_heads: int, value_heads: int,
                 head_size: int, inner_size: int, eps: float):
        self.ctx = ctx
        self.dims = dict(conv_size=conv_size, conv_kernel=conv_kernel, state_size=state_size, key_heads=key_heads,
                         value_heads=value_heads, head_size=head_size, inner_size=inner_size)
        arrays = [np.ascontiguousarray(a, dtype=np.float32) for a in (conv_w, ssm_a, ssm_dt, ssm_norm)]
        h = C.c_void_p()
        ctx.call("fortai_hip_qwen35_recurrent_create", ctx.h, qkv.h, gate.h, alpha.h, beta.h, out.h,
                 _ptr(arrays[0]), arrays[0].nbytes, conv_size, conv_kernel, _ptr(arrays[1]), arrays[1].nbytes,
                 _ptr(arrays[2]), arrays[2].nbytes, _ptr(arrays[3]), arrays[3].nbytes, state_size, key_heads,
                 value_heads, head_size, inner_size, eps, C.byref(h))
        self.h = h

    def reset(self) -> None:
        self.ctx.call("fortai_hip_qwen35_recurrent_reset", self.h)

    def state(self):
        d = self.dims
        gdn = np.empty(d["value_heads"] * d["head_size"] ** 2, dtype=np.float32)
        conv = np.empty((d["conv_kernel"] - 1) * d["conv_size"], dtype=np.float32)
        self.ctx.call("fortai_hip_qwen35_recurrent_state_download", self.h, _ptr(gdn), gdn.nbytes, _ptr(conv),
                      conv.nbytes)
        return gdn, conv

    def set_state(self, gdn: np.ndarray, conv: np.ndarray) -> None:
        gdn = np.ascontiguousarray(gdn, dtype=np.float32)
        conv = np.ascontiguousarray(conv, dtype=np.float32)
        self.ctx.call("fortai_hip_qwen35_recurrent_state_upload", self.h, _ptr(gdn), gdn.nbytes, _ptr(conv),
                      conv.nbytes)

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_qwen35_recurrent_destroy(self.h)
            self.h = None


class Attention:
    """Qwen3.5 gated full-attention layer (fortai_cuda_qwen35_attention)."""

    def __init__(self, ctx: Context, q: Q8Weights, k: Q8Weights, v: Q8Weights, o: Q8Weights, q_norm: np.ndarray,
                 k_norm: np.ndarray, heads: int, kv_heads: int, head_size: int, value_size: int, max_context: int,
                 rope_dim: int, rope_base: float, eps: float):
        self.ctx = ctx
        self.dims = dict(heads=heads, kv_heads=kv_heads, head_size=head_size, value_size=value_size,
                         max_context=max_context)
        qn = np.ascontiguousarray(q_norm, dtype=np.float32)
        kn = np.ascontiguousarray(k_norm, dtype=np.float32)
        h = C.c_void_p()
        ctx.call("fortai_hip_qwen35_attention_create", ctx.h, q.h, k.h, v.h, o.h, _ptr(qn), qn.nbytes, _ptr(kn),
                 kn.nbytes, heads, kv_heads, head_size, value_size, max_context, rope_dim, rope_base, eps,
                 C.byref(h))
        self.h = h

    def reset(self) -> None:
        self.ctx.call("fortai_hip_qwen35_attention_reset", self.h)

    def set_exact_max(self, exact_max: int) -> None:
        """Positions up to which the output keeps the reference's summation
        orders (default 8192); split-K beyond.  Before a decoder is created."""
        self.ctx.call("fortai_hip_qwen35_attention_set_exact_max", self.h, exact_max)

    def set_test_options(self, z_skew: int = 0, force_wide: bool = False) -> None:
        """Test only: shift the Z candidate windows; the wide output kernel for one sequence."""
        self.ctx.call("fortai_hip_qwen35_attention_set_test_options", self.h, z_skew, 1 if force_wide else 0)

    def cache(self, positions: int):
        d = self.dims
        k = np.empty(positions * d["kv_heads"] * d["head_size"], dtype=np.uint16)
        v = np.empty(positions * d["kv_heads"] * d["value_size"], dtype=np.uint16)
        self.ctx.call("fortai_hip_qwen35_attention_cache_download", self.h, _ptr(k), _ptr(v), positions)
        return k, v

    def set_cache(self, k: np.ndarray, v: np.ndarray, positions: int) -> None:
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        self.ctx.call("fortai_hip_qwen35_attention_cache_upload", self.h, _ptr(k), _ptr(v), positions)

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_qwen35_attention_destroy(self.h)
            self.h = None


class Decoder:
    """Fused whole-token decoder (one captured HIP graph per step)."""

    def __init__(self, ctx: Context, recurrent: Sequence[Optional[Recurrent]],
                 attention: Sequence[Optional[Attention]], ffn_gate: Sequence[Q8Weights],
                 ffn_up: Sequence[Q8Weights], ffn_down: Sequence[Q8Weights], attn_norm: Sequence[np.ndarray],
                 post_norm: Sequence[np.ndarray], output_norm: np.ndarray, hidden: int,
                 embedding, output, max_context: int, eps: float, vocab: int):
        self.ctx, self.vocab, self.max_context = ctx, vocab, max_context
        n = len(ffn_gate)

        def harr(items):
            return (C.c_void_p * n)(*[(x.h if x is not None else None) for x in items])

        self._norms = [np.ascontiguousarray(a, dtype=np.float32) for a in list(attn_norm) + list(post_norm)]
        an = (C.c_void_p * n)(*[_ptr(a) for a in self._norms[:n]])
        pn = (C.c_void_p * n)(*[_ptr(a) for a in self._norms[n:]])
        self._onorm = np.ascontiguousarray(output_norm, dtype=np.float32)
        e16 = embedding.h if isinstance(embedding, F16Weights) else None
        e8 = embedding.h if isinstance(embedding, Q8Weights) else None
        o16 = output.h if isinstance(output, F16Weights) else None
        o8 = output.h if isinstance(output, Q8Weights) else None
        h = C.c_void_p()
        ctx.call("fortai_hip_qwen35_decoder_create", ctx.h, n, harr(recurrent), harr(attention), harr(ffn_gate),
                 harr(ffn_up), harr(ffn_down), an, pn, _ptr(self._onorm), hidden, e16, e8, o16, o8, max_context,
                 eps, C.byref(h))
        self.h = h
        self.logits = np.zeros(vocab, dtype=np.float32)

    def reset(self) -> None:
        self.ctx.call("fortai_hip_qwen35_decoder_reset", self.h)

    def set_mode(self, direct: bool = False, matvec_only: bool = False, only: Sequence[str] = ()) -> None:
        """direct: enqueue the kernels every step instead of a graph replay
        (kernel tracing); matvec_only / only: timing probes that enqueue only
        those kernel families ("matvec", "gdn", "attention", "head")."""
        flags = (DECODER_DIRECT if direct else 0) | (DECODER_MATVEC_ONLY if matvec_only else 0)
        for f in only:
            flags |= DECODER_FAMILIES[f]
        self.ctx.call("fortai_hip_qwen35_decoder_set_mode", self.h, flags)

    def forward(self, token: int, position: int, want_logits: bool = True) -> int:
        nxt = np.zeros(1, dtype=np.int64)
        self.ctx.call("fortai_hip_qwen35_decoder_forward", self.h, token, position,
                      _ptr(self.logits) if want_logits else None, _ptr(nxt))
        return int(nxt[0])

    def generate(self, token: int, position: int, steps: int) -> np.ndarray:
        trace = np.zeros(steps, dtype=np.int64)
        self.ctx.call("fortai_hip_qwen35_decoder_generate", self.h, token, position, steps, _ptr(trace))
        return trace

    def replay(self, steps: int) -> None:
        self.ctx.call("fortai_hip_qwen35_decoder_replay", self.h, steps)

    def trace(self, first: int, count: int) -> np.ndarray:
        """The greedy ids chosen at positions first .. first+count-1."""
        out = np.zeros(count, dtype=np.int64)
        self.ctx.call("fortai_hip_qwen35_decoder_trace", self.h, first, count, _ptr(out))
        return out

    def check(self) -> None:
        """Wait for the queued steps; raise if one failed."""
        self.ctx.call("fortai_hip_qwen35_decoder_status", self.h)

    def plan(self):
        """The launches of one step: [(operation, kernel, batch)]."""
        return _plan(self.ctx, "fortai_hip_qwen35_decoder_plan", self.h)

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_qwen35_decoder_destroy(self.h)
            self.h = None


class BatchDecoder:
    """``batch`` independent sequences over one set of layers and weights (one
    captured graph per step, every weight read once for all sequences)."""

    def __init__(self, ctx: Context, batch: int, recurrent: Sequence[Optional[Recurrent]],
                 attention: Sequence[Optional[Attention]], ffn_gate: Sequence[Q8Weights],
                 ffn_up: Sequence[Q8Weights], ffn_down: Sequence[Q8Weights], attn_norm: Sequence[np.ndarray],
                 post_norm: Sequence[np.ndarray], output_norm: np.ndarray, hidden: int,
                 embedding, output, max_context: int, eps: float, vocab: int):
        self.ctx, self.batch, self.vocab, self.max_context = ctx, batch, vocab, max_context
        n = len(ffn_gate)

        def harr(items):
            return (C.c_void_p * n)(*[(x.h if x is not None else None) for x in items])

        self._norms = [np.ascontiguousarray(a, dtype=np.float32) for a in list(attn_norm) + list(post_norm)]
        an = (C.c_void_p * n)(*[_ptr(a) for a in self._norms[:n]])
        pn = (C.c_void_p * n)(*[_ptr(a) for a in self._norms[n:]])
        self._onorm = np.ascontiguousarray(output_norm, dtype=np.float32)
        e16 = embedding.h if isinstance(embedding, F16Weights) else None
        e8 = embedding.h if isinstance(embedding, Q8Weights) else None
        o16 = output.h if isinstance(output, F16Weights) else None
        o8 = output.h if isinstance(output, Q8Weights) else None
        h = C.c_void_p()
        ctx.call("fortai_hip_qwen35_batch_create", ctx.h, batch, n, harr(recurrent), harr(attention),
                 harr(ffn_gate), harr(ffn_up), harr(ffn_down), an, pn, _ptr(self._onorm), hidden, e16, e8, o16, o8,
                 max_context, eps, C.byref(h))
        self.h = h
        self.logits = np.zeros((batch, vocab), dtype=np.float32)

    def _inputs(self, tokens, positions):
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        p = np.ascontiguousarray(positions, dtype=np.int32)
        if t.shape != (self.batch,) or p.shape != (self.batch,):
            raise ValueError(f"need {self.batch} tokens and positions")
        return t, p

    def reset(self) -> None:
        self.ctx.call("fortai_hip_qwen35_batch_reset", self.h)

    def set_mode(self, direct: bool = False) -> None:
        self.ctx.call("fortai_hip_qwen35_batch_set_mode", self.h, DECODER_DIRECT if direct else 0)

    def set_prefill_mode(self, mode: str) -> None:
        """'exact' (default), 'matvec' (same bits) or 'fast' (not bit-exact)."""
        self.ctx.call("fortai_hip_qwen35_batch_set_prefill_mode", self.h, PREFILL_MODES[mode])

    def forward(self, tokens, positions, want_logits: bool = True) -> np.ndarray:
        t, p = self._inputs(tokens, positions)
        nxt = np.zeros(self.batch, dtype=np.int64)
        self.ctx.call("fortai_hip_qwen35_batch_forward", self.h, _ptr(t), _ptr(p),
                      _ptr(self.logits) if want_logits else None, _ptr(nxt))
        return nxt

    def generate(self, tokens, positions, steps: int) -> np.ndarray:
        t, p = self._inputs(tokens, positions)
        trace = np.zeros((self.batch, steps), dtype=np.int64)
        self.ctx.call("fortai_hip_qwen35_batch_generate", self.h, _ptr(t), _ptr(p), steps, _ptr(trace))
        return trace

    def replay(self, steps: int) -> None:
        self.ctx.call("fortai_hip_qwen35_batch_replay", self.h, steps)

    def plan(self, prefill: bool = False):
        """The launches of one batched step (or of the last prefill)."""
        return _plan(self.ctx, "fortai_hip_qwen35_batch_plan", self.h, 1 if prefill else 0)

    def prefill(self, tokens, want_logits: bool = True):
        """Prompt tokens [batch][T] from position 0; returns (next tokens,
        prefill milliseconds); logits of the last prompt token in .logits."""
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        if t.ndim != 2 or t.shape[0] != self.batch:
            raise ValueError(f"need tokens [{self.batch}][T]")
        nxt = np.zeros(self.batch, dtype=np.int64)
        ms = C.c_float()
        self.ctx.call("fortai_hip_qwen35_batch_prefill", self.h, _ptr(t), t.shape[1], _ptr(nxt),
                      _ptr(self.logits) if want_logits else None, C.byref(ms))
        return nxt, ms.value

    def free(self) -> None:
        if self.h:
            self.ctx.lib.fortai_hip_qwen35_batch_destroy(self.h)
            self.h = None
