"""ctypes access to the parity checkers.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline).  The product path (``fortai_amd``) never imports it.

Two checkers live here:

* ``Oracle`` -- ``oracle/liboracle.so``, this repository's C restatement of
  the reference CPU path (``oracle/fortai_oracle.c``).  It travels to the GPU
  box with the tree.
* ``Reference`` -- ``oracle/_ref/``, the reference's own CPU sources
  (``src/backend/cpu/fortai_q8_dot.c``, the Fortran model) compiled by
  ``oracle/Makefile`` in the container that has ``/root/reference``.

How each oracle function is pinned (a check that a plausible mistake fails):

=====================  ===================================================
function               pinned by
=====================  ===================================================
half_to_float          all 65536 fp16 patterns vs numpy float16 (IEEE)
float_to_half          2^32-sample sweep incl. every exponent/tie pattern
                       vs the compiled reference ``fortai_float_to_half``
f32_to_f16_rne         vs numpy astype(float16) (IEEE RNE) on edge sweeps
gguf_fp16_to_real      vs numpy float16 for finite halves; exp 31 -> huge
q8_quantize            reference golden (test_fortai_smoke.f90:221-234);
                       compiled reference bytes; closed-form amax/127 scale
q8_dot / block dots    brute-force integer sums; compiled reference floats
                       bit-exact; smoke goldens 527.9677734375 etc.
gdn_step               smoke golden (test_fortai_smoke.f90:272-281);
                       compiled reference bit-exact; scalar recurrence of
                       fortai_cuda_gdn_ar_bench.cu:165-197 within 2e-5+3e-4|x|
expf (device twin)     orc_expf_restated == host expf on every float of
                       [-103.5, 0] and on samples of (0, 88] (the GPU's
                       expf_libm is the same sequence)
silu / silu_product    |x/(1+e^-x) - silu| <= 2e-5 on [-20,20]
                       (test_fortai_smoke.f90:284-300); compiled reference
rms_norm, l2, rope     closed forms in float64 (tests/test_oracle.py)
attention              brute-force float64 softmax on tiny L
model forward          compiled reference (oracle/_ref/ref_dump) logits,
                       KV caches and GDN/conv states bit-exact; token trace
=====================  ===================================================
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64, _f32, _vp = C.c_int64, C.c_float, C.c_void_p


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)


class Oracle:
    def __init__(self, path: str = LIB):
        if not os.path.exists(path):
            build()
        lib = C.CDLL(path)
        self.lib = lib
        sig = {
            "orc_half_to_float": (_f32, [C.c_uint16]),
            "orc_float_to_half": (C.c_uint16, [_f32]),
            "orc_f32_to_f16_rne": (C.c_uint16, [_f32]),
            "orc_gguf_fp16_to_real": (_f32, [C.c_uint16]),
            "orc_q8_quantize": (None, [_f32p, _i8p, _f32p, _i64]),
            "orc_q8_dequantize_row": (None, [_i8p, _f32p, _i64]),
            "orc_q8_dot": (_f32, [_i8p, _i8p, _f32p, _i64, _i64]),
            "orc_q8_block_dots": (None, [_i8p, _i8p, _i64, _i64, _i32p]),
            "orc_q8_matvec": (None, [_i8p, _i64, _i64, _f32p, _f32p, _i8p, _f32p]),
            "orc_expf_poly": (_f32, [_f32]),
            "orc_silu": (None, [_f32p, _i64]),
            "orc_silu_product": (None, [_f32p, _f32p, _i64]),
            "orc_gdn_step": (None, [_f32p, _f32p, _f32p, _f32p, _f32, _f32, _i64, _f32, _f32p]),
            "orc_rms_norm": (None, [_f32p, _f32p, _f32, _f32p, _i64]),
            "orc_normalize_slice": (None, [_f32p, _i64, _f32, _f32p]),
            "orc_l2_normalize_slice": (None, [_f32p, _i64, _f32]),
            "orc_rms_slice": (_f32, [_f32p, _i64, _f32]),
            "orc_sigmoid": (_f32, [_f32]),
            "orc_softplus": (_f32, [_f32]),
            "orc_rope_cos_sin": (None, [_i64, _i64, _i64, _f32, C.POINTER(_f32), C.POINTER(_f32)]),
            "orc_apply_rope": (None, [_f32p, _i64, _i64, _i64, _i64, _f32]),
            "orc_attention_apply": (None, [_f32p, _u16p, _u16p, _i64, _i64, _i64, _i64, _i64, _f32p, _f32p]),
            "orc_attention_core_step": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _u16p, _u16p, _i64, _i64,
                                               _i64, _i64, _i64, _i64, _f32, _f32, _f32p, _f32p]),
            "orc_gdn_core_step": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64,
                                         _i64, _i64, _i64, _i64, _f32, _f32p, _f32p]),
            "orc_model_open": (_vp, [C.c_char_p, _i64]),
            "orc_model_close": (None, [_vp]),
            "orc_model_reset": (None, [_vp]),
            "orc_model_forward": (C.c_int, [_vp, _i64, _i64, _f32p]),
            "orc_argmax": (_i64, [_f32p, _i64]),
            "orc_model_dims": (_i64, [_vp, _i64p, _i64]),
            "orc_model_hidden": (C.POINTER(_f32), [_vp]),
            "orc_model_gdn_state": (C.POINTER(_f32), [_vp, _i64]),
            "orc_model_conv_state": (C.POINTER(_f32), [_vp, _i64]),
            "orc_model_kcache": (C.POINTER(C.c_uint16), [_vp, _i64]),
            "orc_model_vcache": (C.POINTER(C.c_uint16), [_vp, _i64]),
            "orc_threads": (C.c_int, []),
            "orc_float_to_half_mismatches": (_i64, [_vp, C.c_uint64, C.c_uint64]),
            "orc_float_to_half_array": (None, [_f32p, _u16p, _i64]),
            "orc_f32_to_f16_rne_array": (None, [_f32p, _u16p, _i64]),
            "orc_half_to_float_array": (None, [_u16p, _f32p, _i64]),
            "orc_gguf_fp16_to_real_array": (None, [_u16p, _f32p, _i64]),
            "orc_expf_restated": (_f32, [_f32]),
            "orc_expf_restated_mismatches": (_i64, [C.c_uint32, C.c_uint32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args

    def __getattr__(self, name):
        return getattr(self.lib, "orc_" + name)

    # ---- numpy conveniences
    def quantize(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.size // 32 * 34, dtype=np.int8)
        s = np.zeros(x.size // 32, dtype=np.float32)
        self.lib.orc_q8_quantize(x, q, s, x.size)
        return q, s

    def matvec(self, w34: np.ndarray, rows: int, width: int, x: np.ndarray) -> np.ndarray:
        out = np.zeros(rows, dtype=np.float32)
        q = np.zeros(width // 32 * 34, dtype=np.int8)
        s = np.zeros(width // 32, dtype=np.float32)
        self.lib.orc_q8_matvec(np.ascontiguousarray(w34).view(np.int8).reshape(-1), rows, width,
                               np.ascontiguousarray(x, dtype=np.float32), out, q, s)
        return out

    def block_dots(self, w34: np.ndarray, q: np.ndarray, rows: int, nb: int) -> np.ndarray:
        out = np.zeros(rows * nb, dtype=np.int32)
        self.lib.orc_q8_block_dots(np.ascontiguousarray(w34).view(np.int8).reshape(-1), q, rows, nb, out)
        return out.reshape(rows, nb)


class OracleModel:
    """The restated Qwen3.5 CPU decode step over a GGUF file."""

    DIM_NAMES = ["hidden", "vocab", "layers", "ffn", "heads", "kv_heads", "head_size", "value_size",
                 "rope_dim", "conv_kernel", "state_size", "key_heads", "value_heads", "inner", "gdn_head",
                 "conv_size", "interval", "max_context"]

    def __init__(self, oracle: Oracle, path: str, max_context: int):
        self.o = oracle
        self.h = oracle.lib.orc_model_open(path.encode(), max_context)
        if not self.h:
            raise RuntimeError(f"oracle could not open {path}")
        d = np.zeros(len(self.DIM_NAMES), dtype=np.int64)
        oracle.lib.orc_model_dims(self.h, d, d.size)
        self.dims = dict(zip(self.DIM_NAMES, (int(v) for v in d)))
        self.logits = np.zeros(self.dims["vocab"], dtype=np.float32)

    def close(self):
        if self.h:
            self.o.lib.orc_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        self.o.lib.orc_model_reset(self.h)

    def forward(self, token: int, position: int) -> np.ndarray:
        if self.o.lib.orc_model_forward(self.h, token, position, self.logits) != 0:
            raise ValueError("invalid token or position")
        return self.logits

    def greedy(self, token: int, steps: int, start: int = 0, keep_logits: bool = False):
        trace, all_logits = [], []
        for p in range(start, start + steps):
            logits = self.forward(token, p)
            token = int(self.o.lib.orc_argmax(logits, logits.size))
            trace.append(token)
            if keep_logits:
                all_logits.append(logits.copy())
        return (trace, np.array(all_logits)) if keep_logits else trace

    def _arr(self, ptr, n, dtype):
        return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)

    def kcache(self, layer: int) -> np.ndarray:
        d = self.dims
        return self._arr(self.o.lib.orc_model_kcache(self.h, layer),
                         d["max_context"] * d["kv_heads"] * d["head_size"], np.uint16)

    def vcache(self, layer: int) -> np.ndarray:
        d = self.dims
        return self._arr(self.o.lib.orc_model_vcache(self.h, layer),
                         d["max_context"] * d["kv_heads"] * d["value_size"], np.uint16)

    def gdn_state(self, layer: int) -> np.ndarray:
        d = self.dims
        return self._arr(self.o.lib.orc_model_gdn_state(self.h, layer),
                         d["gdn_head"] ** 2 * d["value_heads"], np.float32)

    def conv_state(self, layer: int) -> np.ndarray:
        d = self.dims
        return self._arr(self.o.lib.orc_model_conv_state(self.h, layer),
                         (d["conv_kernel"] - 1) * d["conv_size"], np.float32)


class Reference:
    """The reference's own CPU code, compiled by oracle/Makefile into oracle/_ref."""

    def __init__(self, ref_dir: str = REF_DIR):
        self.dir = ref_dir
        self.lib: Optional[C.CDLL] = None
        path = os.path.join(ref_dir, "libfortai_q8_dot.so")
        if os.path.exists(path):
            lib = C.CDLL(path)
            lib.fortai_float_to_half.restype = C.c_uint16
            lib.fortai_float_to_half.argtypes = [_f32]
            lib.fortai_q8_quantize.restype = None
            lib.fortai_q8_quantize.argtypes = [_f32p, _i8p, _f32p, _i64]
            lib.fortai_q8_dot.restype = _f32
            lib.fortai_q8_dot.argtypes = [_i8p, _i8p, _f32p, _i64, _i64]
            lib.fortai_q8_dequantize_row.restype = None
            lib.fortai_q8_dequantize_row.argtypes = [_i8p, _f32p, _i64]
            lib.fortai_gdn_step.restype = None
            lib.fortai_gdn_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32, _f32, _i64, _f32, _f32p]
            lib.fortai_silu.restype = None
            lib.fortai_silu.argtypes = [_f32p, _i64]
            lib.fortai_silu_product.restype = None
            lib.fortai_silu_product.argtypes = [_f32p, _f32p, _i64]
            self.lib = lib

    @property
    def available(self) -> bool:
        return self.lib is not None

    def exe(self, name: str) -> str:
        return os.path.join(self.dir, name)

    def has(self, name: str) -> bool:
        return os.path.exists(self.exe(name))

    def dump(self, model: str, token: int, steps: int, context: int, out_dir: str,
             state: bool = False, threads: Optional[int] = None, keep_logits: bool = False) -> dict:
        """keep_logits: leave the logits on disk (out_dir/logits.f32) instead
        of loading them (a long trace's logits are gigabytes)."""
        os.makedirs(out_dir, exist_ok=True)
        env = dict(os.environ)
        if threads:
            env["OMP_NUM_THREADS"] = str(threads)
        subprocess.run([self.exe("ref_dump"), model, str(token), str(steps), str(context), out_dir,
                        "1" if state else "0"], check=True, env=env, stdout=subprocess.DEVNULL)
        if keep_logits:
            return {"tokens": np.fromfile(os.path.join(out_dir, "tokens.i64"), dtype=np.int64)}
        logits = np.fromfile(os.path.join(out_dir, "logits.f32"), dtype=np.float32).reshape(steps, -1)
        tokens = np.fromfile(os.path.join(out_dir, "tokens.i64"), dtype=np.int64)
        return {"logits": logits, "tokens": tokens}
