"""Writer for the .fgm layout (convert/fgm.py:1-16): magic b"FASTGEM1", u32
little-endian header length, compact JSON header {arch, config, meta,
tensors: {name: {dtype, shape, offset, nbytes, meta}}}, tensor blobs 64-byte
aligned at absolute offsets after the header.  Used for synthetic model files
(tests, benchmarks); real files come from the reference's converter."""
from __future__ import annotations

import json
import struct

MAGIC = b"FASTGEM1"
ALIGN = 64


def _pad(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


def write_fgm(path, config: dict, tensors, meta: dict | None = None, arch: str = "gemma3n"):
    """tensors: iterable of (name, data: bytes | ndarray, dtype, shape, meta).
    Returns the header's tensor table."""
    entries, blobs = {}, []
    for name, data, dtype, shape, tmeta in tensors:
        b = data.tobytes() if hasattr(data, "tobytes") else bytes(data)
        entries[name] = {"dtype": dtype, "shape": list(shape), "offset": 0, "nbytes": len(b),
                         "meta": tmeta or {}}
        blobs.append((name, b))
    probe = json.dumps({"arch": arch, "config": config, "meta": meta or {}, "tensors": entries},
                       separators=(",", ":")).encode()
    reserve = len(probe) + 24 * len(entries) + 256      # room for the final offsets
    cursor = _pad(12 + reserve)
    for name, b in blobs:
        entries[name]["offset"] = cursor
        cursor = _pad(cursor + len(b))
    header = json.dumps({"arch": arch, "config": config, "meta": meta or {}, "tensors": entries},
                        separators=(",", ":")).encode()
    assert len(header) <= reserve
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<I", len(header)) + header)
        for name, b in blobs:
            f.seek(entries[name]["offset"])
            f.write(b)
    return entries
