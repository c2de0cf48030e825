"""Host-side logic that needs no GPU: the GGUF reader/writer, the synthetic
model generator, layout arithmetic, the bench's byte model, and the C ABI
library's exports (loaded, never called)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
from types import SimpleNamespace

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fortai_hip_backend.h")
LIB = os.path.join(ROOT, "fortai_amd", "lib", "libfortai_hip.so")


def header_symbols() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fortai_hip_\w+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    """Every entry point of backend/cuda/fortai_cuda_backend.h has a
    fortai_hip_* counterpart (same argument order, hip prefix)."""
    syms = set(header_symbols())
    # the entry points of backend/cuda/fortai_cuda_backend.h:22-152
    mirrored = [
        "q8_context_capture_begin", "q8_context_capture_end", "q8_context_create", "q8_context_destroy",
        "q8_context_graph_launch", "q8_context_set_position", "q8_device_buffer_create",
        "q8_device_buffer_destroy", "q8_device_buffer_download", "q8_device_buffer_upload",
        "q8_device_buffer_upload_ptr", "q8_ffn_device", "q8_ffn_host", "q8_last_error",
        "q8_matvec_device_f32", "q8_matvec_host", "q8_matvec_host_pair", "q8_matvec_host_triplet",
        "q8_matvec_host_triplet_contiguous", "q8_matvec_resident", "q8_weights_destroy",
        "q8_weights_upload", "qwen35_add_device", "qwen35_attention_create", "qwen35_attention_destroy",
        "qwen35_attention_reset", "qwen35_attention_run_device", "qwen35_copy_device",
        "qwen35_embedding_device", "qwen35_recurrent_create", "qwen35_recurrent_destroy",
        "qwen35_recurrent_reset", "qwen35_recurrent_run", "qwen35_recurrent_run_device",
        "qwen35_rms_norm_device",
    ]
    missing = [m for m in mirrored if "fortai_hip_" + m not in syms]
    assert not missing, missing


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        subprocess.run(["python", "-c", "from fortai_amd import build; build.build()"], cwd=ROOT, check=True)
    lib = ctypes.CDLL(LIB)  # loading initialises no device
    missing = [s for s in header_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    from fortai_amd import backend
    assert set(backend.exported_symbols()) <= set(header_symbols())
    assert set(header_symbols()) <= set(backend.exported_symbols())


def test_gguf_roundtrip(tmp_path):
    from fortai_amd import gguf
    path = str(tmp_path / "t.gguf")
    w = gguf.Writer(path)
    w.add_meta("general.architecture", gguf.GGUF_STRING, "qwen35")
    w.add_meta("qwen35.block_count", gguf.GGUF_UINT32, 3)
    w.add_meta("qwen35.rope.freq_base", gguf.GGUF_FLOAT32, 1.0e7)
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 64)).astype(np.float32)
    b = rng.standard_normal((3, 96)).astype(np.float16)
    from fortai_amd import synth
    c = synth.q8_blocks(rng, 7, 64)
    w.add_tensor("a", (64, 5), gguf.GGML_TYPE_F32)
    w.add_tensor("b", (96, 3), gguf.GGML_TYPE_F16)
    w.add_tensor("c", (64, 7), gguf.GGML_TYPE_Q8_0)
    w.write({"a": a, "b": b, "c": c}.__getitem__)
    f = gguf.read(path)
    assert f.meta_int("qwen35.block_count") == 3
    assert f.meta_real("qwen35.rope.freq_base", 0.0) == np.float32(1.0e7)
    assert np.array_equal(f.tensor("a").as_f32().reshape(5, 64), a)
    assert np.array_equal(f.tensor("b").as_f16_bits().reshape(3, 96), b.view(np.uint16))
    t = f.tensor("c")
    assert (t.rows, t.width) == (7, 64)
    assert np.array_equal(np.frombuffer(t.data, dtype=np.uint8)[: c.size], c.reshape(-1))


def test_synth_is_deterministic_and_complete(tmp_path):
    from fortai_amd import gguf, synth, qwen35
    cfg = synth.CONFIGS["qwen35-tiny"]
    p1, p2 = str(tmp_path / "1.gguf"), str(tmp_path / "2.gguf")
    synth.write_model(p1, cfg)
    synth.write_model(p2, cfg)
    assert open(p1, "rb").read() == open(p2, "rb").read()
    f = gguf.read(p1)
    d = qwen35.read_dims(f)
    assert (d.hidden, d.layers, d.vocab, d.heads, d.kv_heads) == (cfg.hidden, cfg.layers, cfg.vocab,
                                                                 cfg.heads, cfg.kv_heads)
    for name, shape, ggml_type in synth.tensor_specs(cfg):
        t = f.tensor(name)
        assert t is not None and tuple(t.shape) == tuple(shape) and t.ggml_type == ggml_type, name
    assert f.tensor("output.weight") is None  # tied LM head
    # ssm_a < 0 so every decay factor exp(a * softplus(.)) is below one
    for layer in range(cfg.layers):
        if cfg.recurrent(layer):
            assert np.all(f.tensor(f"blk.{layer}.ssm_a").as_f32() < 0)


def test_q8_blocks_distribution():
    from fortai_amd import synth
    b = synth.q8_blocks(np.random.default_rng(1), 64, 1024).reshape(64, 32, 34)
    q = b[:, :, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127
    s = np.abs(b[:, :, :2].copy().view(np.float16).astype(np.float32))
    assert s.min() >= 1e-3 * 0.999 and s.max() <= 1e-1 * 1.001


def test_bytes_per_token_matches_the_byte_model():
    """1,079.4 MB + 12,288 B per cached position for the 0.8B shape."""
    import bench
    from fortai_amd import synth
    c = synth.CONFIGS["qwen35-0.8b"]
    d = SimpleNamespace(hidden=c.hidden, layers=c.layers, ffn=c.ffn, heads=c.heads, kv_heads=c.kv_heads,
                        head_size=c.head_size, value_size=c.value_size, conv_size=c.conv_size,
                        inner=c.gdn_inner, value_heads=c.gdn_value_heads, gdn_head=c.gdn_head,
                        conv_kernel=c.conv_kernel, vocab=c.vocab, interval=c.interval)
    b0 = bench.bytes_per_token(d, 0)
    assert abs(b0 / 1e6 - 1079.4) < 0.1
    assert bench.bytes_per_token(d, 4096) - b0 == 12288 * 4096


def test_bench_refuses_several_gpus():
    r = subprocess.run(["python", os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_product_has_no_oracle_dependency():
    """The shipped package neither imports nor links the parity checker."""
    pkg = os.path.join(ROOT, "fortai_amd")
    for dirpath, _, files in os.walk(pkg):
        for name in files:
            if name.endswith((".py", ".hip", ".h", ".cpp", ".f90")):
                text = open(os.path.join(dirpath, name), errors="ignore").read()
                for needle in ("from oracle", "import oracle", "liboracle", "orc_", "_ref/"):
                    assert needle not in text, (name, needle)
                assert "/root/reference" not in text, name


def test_backend_load_fails_loudly_without_library(tmp_path):
    from fortai_amd import backend
    saved = backend._lib
    backend._lib = None
    try:
        with pytest.raises(FileNotFoundError):
            backend.load(str(tmp_path / "missing.so"))
    finally:
        backend._lib = saved


def test_weak_stub_covers_the_header(tmp_path):
    """fortai_hip_stub.c defines every declared entry point (weak) and fails
    each call with FORTAI_HIP_RUNTIME_ERROR."""
    so = str(tmp_path / "libstub.so")
    subprocess.run(["gcc", "-shared", "-fPIC", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "fortai_amd", "fortran", "fortai_hip_stub.c"), "-o", so], check=True)
    lib = ctypes.CDLL(so)
    assert all(hasattr(lib, s) for s in header_symbols())
    lib.fortai_hip_q8_context_create.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    h = ctypes.c_void_p()
    assert lib.fortai_hip_q8_context_create(0, ctypes.byref(h)) == 2
    lib.fortai_hip_q8_last_error.restype = ctypes.c_char_p
    assert b"without the HIP backend" in lib.fortai_hip_q8_last_error(None)
    # as src/backend/cpu/fortai_cuda_stub.c:13-23: a failed create leaves its
    # out-handle NULL (a caller's later destroy is then a no-op) ...
    for name, nargs in (("fortai_hip_q8_context_create", 1), ("fortai_hip_q8_weights_upload", 5),
                        ("fortai_hip_f16_weights_upload", 5), ("fortai_hip_q8_device_buffer_create", 2),
                        ("fortai_hip_q8_weights_upload_packed", 5)):
        h = ctypes.c_void_p(0x1234)
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.c_void_p] * nargs + [ctypes.POINTER(ctypes.c_void_p)]
        assert fn(*([None] * nargs), ctypes.byref(h)) == 2, name
        assert h.value is None, name
    # ... and every destroy succeeds, NULL included
    destroys = [s for s in header_symbols() if s.endswith("_destroy")]
    assert len(destroys) >= 8
    for name in destroys:
        fn = getattr(lib, name)
        nargs = 2 if name == "fortai_hip_q8_device_buffer_destroy" else 1
        fn.argtypes = [ctypes.c_void_p] * nargs
        assert fn(*([None] * nargs)) == 0, name


def test_pack_key_and_cache_path(tmp_path):
    """pack_key_t / cache_path as src/fortai_cache.f90:6-43 defines them, and
    the pack file round trip (records, digest check)."""
    import numpy as np
    from fortai_amd import pack_cache as pc
    key = pc.PackKey(model="qwen35-0.8b", backend="hip-gfx950", variant="q8-lanes", abi_version=3)
    assert key.is_valid()
    assert pc.cache_path("/cache", key) == "/cache/qwen35-0.8b/hip-gfx950-q8-lanes-abi3.pack"
    for bad in (pc.PackKey(), pc.PackKey("m", "b", " ", 1), pc.PackKey("m", "b", "v", 0)):
        assert not bad.is_valid()
        assert pc.cache_path("/cache", bad) == "/cache/invalid.pack"
    recs = {"blk.0.ffn_up.weight": (3, 64, np.arange(200, dtype=np.uint8)),
            "output.weight": (9, 32, np.zeros(7, dtype=np.uint8))}
    path = str(tmp_path / "m" / "p.pack")
    pc.write(path, b"d" * 32, recs)
    got = pc.read(path, b"d" * 32)
    assert set(got) == set(recs)
    for n, (r, w, a) in recs.items():
        assert got[n][0] == r and got[n][1] == w and np.array_equal(got[n][2], a)
    assert pc.read(path, b"e" * 32) is None          # made from another GGUF
    assert pc.read(str(tmp_path / "none.pack"), b"d" * 32) is None


def test_fast_division_matches_integer_division(tmp_path):
    """fortai_amd/csrc/fastdiv.h (the device kernels' division by launch-fixed
    divisors) against C's / and %: every divisor 1..1024 with every dividend
    below 2^16, and 2^22 pseudo-random dividends below 2^31 per divisor up to
    2^20 in powers of two and their neighbours."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "fd.cpp"
    src.write_text(r'''
#define __host__
#define __device__
#include "fastdiv.h"
#include <cstdio>
using namespace fortai_hip;
static int check(uint32_t d, uint32_t n) {
    const FastDiv f = fast_div(d);
    return div((int)n, f) != (int)(n / d) || mod((int)n, f) != (int)(n % d);
}
int main() {
    long bad = 0;
    for (uint32_t d = 1; d <= 1024; ++d)
        for (uint32_t n = 0; n < 65536; ++n) bad += check(d, n);
    uint32_t s = 0x6f727461u;
    for (uint32_t e = 0; e <= 20; ++e)
        for (int k = -1; k <= 1; ++k) {
            const uint32_t d = (1u << e) + k;
            if (d == 0) continue;
            for (int i = 0; i < (1 << 18); ++i) {
                s ^= s << 13; s ^= s >> 17; s ^= s << 5;
                bad += check(d, s & 0x7fffffffu);
            }
            bad += check(d, 0x7fffffffu) + check(d, 0x7ffffffeu);
        }
    printf("%ld\n", bad);
    return bad != 0;
}
''')
    exe = tmp_path / "fd"
    subprocess.run([gxx, "-O2", "-I", os.path.join(ROOT, "fortai_amd", "csrc"), str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
