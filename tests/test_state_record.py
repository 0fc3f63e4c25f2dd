"""CPU checks of the streaming-state record (bdh_state_record_info reads only
the header, no device): a record written from the documented layout by an
independent Python writer is read back, and malformed files are refused.
The Python CRC32C is pinned by the standard check value."""
import ctypes

import numpy as np

from tests import staterec


def test_crc32c_check_value():
    # The CRC-32C catalogue check value of the ASCII string "123456789".
    assert staterec.crc32c(b"123456789") == 0xE3069283


def _info(path, max_layers=8):
    from burn_dragon_amd import _lib
    lib = _lib.load()
    pos, n = ctypes.c_int64(), ctypes.c_int32()
    descs = (_lib.BdhLayerStateDesc * max_layers)()
    st = lib.bdh_state_record_info(str(path).encode(), ctypes.byref(pos), ctypes.byref(n), descs,
                                   max_layers)
    return st, pos.value, n.value, descs


def test_info_reads_a_python_written_record(tmp_path):
    from burn_dragon_amd import _lib
    rng = np.random.default_rng(1)
    path = tmp_path / "state.bdh"
    staterec.write_record(path, 1056, [(rng.standard_normal((2, 4, 16, 8)).astype(np.float32), 1, 1),
                                       (None, 0, 1),
                                       (rng.standard_normal((2, 4, 16, 8)).astype(np.float32), 1, 0)])
    st, pos, n, d = _info(path)
    assert st == _lib.BDH_OK, _lib.last_error()
    assert (pos, n) == (1056, 3)
    assert (d[0].batch, d[0].heads, d[0].latent, d[0].embd) == (2, 4, 16, 8)
    assert (d[1].batch, d[1].heads, d[1].latent, d[1].embd) == (0, 0, 0, 0)
    assert (d[1].persist_sequence_state, d[1].retain_terminal_sequence_state) == (0, 1)
    assert (d[2].persist_sequence_state, d[2].retain_terminal_sequence_state) == (1, 0)


def test_info_refuses_malformed_records(tmp_path):
    from burn_dragon_amd import _lib
    bad = tmp_path / "bad.bdh"
    bad.write_bytes(b"NOTARECORD" + bytes(64))
    assert _info(bad)[0] == _lib.BDH_EINVAL and "magic" in _lib.last_error()
    short = tmp_path / "short.bdh"
    short.write_bytes(staterec.MAGIC + b"\x01\x00")
    assert _info(short)[0] == _lib.BDH_EINVAL
    good = tmp_path / "good.bdh"
    staterec.write_record(good, 3, [(np.zeros((1, 1, 2, 2), np.float32), 1, 1)] * 2)
    assert _info(good, max_layers=1)[0] == _lib.BDH_EINVAL  # layers array too short
    assert _info(tmp_path / "missing.bdh")[0] == _lib.BDH_EINVAL
