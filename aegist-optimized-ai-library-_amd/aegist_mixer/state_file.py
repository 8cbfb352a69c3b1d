"""Saved-state file framing (the engine's Lm::save_state / load_state, aegist_rs/src/next.rs:
2442-2578): the 8 bytes ``AEGSTATE``, the header length as a little-endian u64, a JSON header
``{"key": <state key or null>, "toks": [token ids]}``, then the state payload (the pieces
written by aegist_stack_save_state, in layer order). Host-side bytes only; nothing here touches
the device."""
from __future__ import annotations

import json
import os
import struct
from pathlib import Path

MAGIC = b"AEGSTATE"


class StateFileError(ValueError):
    pass


def pack_header(key: str | None, toks: list[int]) -> bytes:
    head = json.dumps({"key": key, "toks": [int(t) for t in toks]}, separators=(",", ":")).encode()
    return MAGIC + struct.pack("<Q", len(head)) + head


def write(path, key: str | None, toks: list[int], payload: bytes) -> None:
    """Write atomically: a .tmp file beside the target, flushed, then renamed over it."""
    path = Path(path)
    tmp = path.with_suffix(".tmp")
    with open(tmp, "wb") as f:
        f.write(pack_header(key, toks))
        f.write(payload)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def read(path, key: str | None) -> tuple[list[int], bytes]:
    """(token ids, payload). Raises StateFileError if the file is not a saved state, was saved
    under another key, or holds no tokens."""
    path = Path(path)
    with open(path, "rb") as f:
        magic = f.read(16)
        if len(magic) < 16 or magic[:8] != MAGIC:
            raise StateFileError(f"{path}: not a saved state")
        (hlen,) = struct.unpack("<Q", magic[8:])
        head_raw = f.read(hlen)
        if len(head_raw) != hlen:
            raise StateFileError(f"{path}: truncated header")
        try:
            head = json.loads(head_raw)
        except json.JSONDecodeError as e:
            raise StateFileError(f"{path}: {e}") from None
        if head.get("key") != key:
            raise StateFileError(f"{path}: saved by another brain")
        toks = [int(t) for t in head.get("toks") or [] if isinstance(t, int)]
        if not toks:
            raise StateFileError(f"{path}: no tokens")
        return toks, f.read()
