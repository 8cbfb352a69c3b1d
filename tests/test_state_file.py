"""CPU checks of the saved-state file framing (engine next.rs:2442-2578)."""
import json
import struct

import pytest

from aegist_mixer import state_file


def test_round_trip_and_layout(tmp_path):
    p = tmp_path / "a.state"
    state_file.write(p, "brain-1", [5, 6, 7], b"\x01\x02\x03")
    raw = p.read_bytes()
    assert raw[:8] == b"AEGSTATE"
    (n,) = struct.unpack("<Q", raw[8:16])
    assert json.loads(raw[16:16 + n]) == {"key": "brain-1", "toks": [5, 6, 7]}
    assert raw[16 + n:] == b"\x01\x02\x03"
    assert state_file.read(p, "brain-1") == ([5, 6, 7], b"\x01\x02\x03")
    assert not (tmp_path / "a.tmp").exists()


def test_rejections(tmp_path):
    p = tmp_path / "b.state"
    state_file.write(p, None, [1], b"")
    assert state_file.read(p, None) == ([1], b"")
    with pytest.raises(state_file.StateFileError, match="another brain"):
        state_file.read(p, "x")
    p.write_bytes(b"NOTSTATE" + bytes(8))
    with pytest.raises(state_file.StateFileError, match="not a saved state"):
        state_file.read(p, None)
    p.write_bytes(state_file.MAGIC + struct.pack("<Q", 100) + b"{}")
    with pytest.raises(state_file.StateFileError, match="truncated"):
        state_file.read(p, None)
    state_file.write(p, None, [], b"")
    with pytest.raises(state_file.StateFileError, match="no tokens"):
        state_file.read(p, None)
