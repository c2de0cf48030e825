"""Repacked-weight cache keyed like the reference's pack files.

The reference names a pack file by model, backend, variant and ABI version
(``src/fortai_cache.f90:6-31``: ``pack_key_t``, ``cache_path``); this module
keeps the same key and path rule and stores, per model, the resident planes
of every Q8_0 matrix as this backend repacks them at upload, so a later load
uploads them directly (``fortai_hip_q8_weights_upload_packed``) instead of
repacking.

File format (this backend's own): magic ``FHIPPACK``, u32 format version,
32-byte SHA-256 of the first MiB of the GGUF it was made from, u32 record
count; then per record: u32 name length, name (UTF-8), u32 rows, u32 width,
u64 byte count, the planes.  A pack whose digest differs from the GGUF being
loaded is ignored.
"""

from __future__ import annotations

import hashlib
import os
import struct
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

MAGIC = b"FHIPPACK"
FORMAT = 1


@dataclass
class PackKey:
    """pack_key_t (src/fortai_cache.f90:6-13)."""
    model: str = ""
    backend: str = ""
    variant: str = ""
    abi_version: int = 1

    def is_valid(self) -> bool:
        """pack_key_is_valid (:32-43): every field set, ABI version positive."""
        return bool(self.model.strip() and self.backend.strip() and self.variant.strip()) and self.abi_version > 0


def cache_path(root: str, key: PackKey) -> str:
    """cache_path (:17-30): root/model/backend-variant-abiN.pack, or
    root/invalid.pack for an invalid key."""
    root = root.rstrip()
    if not key.is_valid():
        return root + "/invalid.pack"
    return f"{root}/{key.model.strip()}/{key.backend.strip()}-{key.variant.strip()}-abi{key.abi_version}.pack"


def gguf_digest(path: str) -> bytes:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read(1 << 20)).digest()


def model_key(gguf_path: str) -> PackKey:
    """This backend's key for a GGUF: the file's stem and size, the
    resident-layout variant and its version."""
    stem = os.path.splitext(os.path.basename(gguf_path))[0]
    return PackKey(model=f"{stem}-{os.path.getsize(gguf_path):x}", backend="hip-gfx950", variant="q8-lanes",
                   abi_version=1)


def write(path: str, digest: bytes, records: Dict[str, Tuple[int, int, np.ndarray]]) -> None:
    os.makedirs(os.path.dirname(path), exist_ok=True)
    tmp = path + ".part"
    with open(tmp, "wb") as f:
        f.write(MAGIC + struct.pack("<I", FORMAT) + digest + struct.pack("<I", len(records)))
        for name, (rows, width, planes) in records.items():
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb + struct.pack("<IIQ", rows, width, planes.nbytes))
            f.write(np.ascontiguousarray(planes).tobytes())
    os.replace(tmp, path)


def read(path: str, digest: bytes) -> Optional[Dict[str, Tuple[int, int, np.ndarray]]]:
    """The records of a pack made from the same GGUF, else None."""
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        head = f.read(len(MAGIC) + 4 + 32 + 4)
        if len(head) < len(MAGIC) + 40 or head[:len(MAGIC)] != MAGIC:
            return None
        (fmt,) = struct.unpack("<I", head[len(MAGIC):len(MAGIC) + 4])
        if fmt != FORMAT or head[len(MAGIC) + 4:len(MAGIC) + 36] != digest:
            return None
        (count,) = struct.unpack("<I", head[-4:])
        out = {}
        for _ in range(count):
            (n,) = struct.unpack("<I", f.read(4))
            name = f.read(n).decode()
            rows, width, nbytes = struct.unpack("<IIQ", f.read(16))
            out[name] = (rows, width, np.frombuffer(f.read(nbytes), dtype=np.uint8))
        return out
