"""The state record's documented file layout, written from Python (the
layout is data: magic, version, layer entries, CRC32C), so that tests can
check the library against an independent writer and checksum."""
import struct

import numpy as np

MAGIC = b"BDHRHO01"
ALIGN = 4096


def crc32c(data: bytes, crc: int = 0) -> int:
    """CRC-32C (Castagnoli, reflected polynomial 0x82F63B78), bitwise."""
    crc ^= 0xFFFFFFFF
    table = _table()
    for b in data:
        crc = table[(crc ^ b) & 0xFF] ^ (crc >> 8)
    return crc ^ 0xFFFFFFFF


_TABLE = None


def _table():
    global _TABLE
    if _TABLE is None:
        t = []
        for i in range(256):
            c = i
            for _ in range(8):
                c = (c >> 1) ^ 0x82F63B78 if c & 1 else c >> 1
            t.append(c)
        _TABLE = t
    return _TABLE


def write_record(path, position, layers):
    """layers: list of (rho f32 array [B,H,N,D] or None, persist, retain)."""
    n = len(layers)
    off = -(-(24 + 64 * n) // ALIGN) * ALIGN
    entries, blobs = [], []
    for rho, persist, retain in layers:
        if rho is None:
            entries.append(struct.pack("<4q2i2Q2I", 0, 0, 0, 0, persist, retain, 0, 0, 0, 0))
            continue
        blob = np.ascontiguousarray(rho, np.float32).tobytes()
        entries.append(struct.pack("<4q2i2Q2I", *rho.shape, persist, retain, off, len(blob),
                                   crc32c(blob), 0))
        blobs.append((off, blob))
        off = -(-(off + len(blob)) // ALIGN) * ALIGN
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<IIq", 1, n, position) + b"".join(entries))
        for o, blob in blobs:
            f.seek(o)
            f.write(blob)
