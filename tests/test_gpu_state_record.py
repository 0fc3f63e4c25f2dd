"""Streaming-state record on the GPU: a model state saved and loaded back is
bit-identical, decoding continues from the loaded state exactly as from the
live one, a record written by the independent Python writer loads (so the
library's CRC32C and layout agree with it), and a corrupted block is
refused."""
import numpy as np
import pytest

from tests import staterec
from tests.gpu_util import announce, dev, host, need_gpu

pytestmark = pytest.mark.gpu


def _model(torch, bd, rng):
    V, D, H, N, L = 256, 64, 2, 256, 3
    enc = (rng.standard_normal((1, H, D, N)) * 0.05).astype(np.float32)
    encv = (rng.standard_normal((1, H, D, N)) * 0.05).astype(np.float32)
    dec = (rng.standard_normal((H * N, D)) * 0.05).astype(np.float32)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    head = (rng.standard_normal((D, V)) * 0.02).astype(np.float32)
    return bd.pack_model(dev(torch, embed), dev(torch, enc), dev(torch, encv), dev(torch, dec),
                         dev(torch, head), L)


def test_save_load_roundtrip_and_continuation(tmp_path):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(31)
    w = _model(torch, bd, rng)
    tokens = dev(torch, rng.integers(0, 256, (2, 24)).astype(np.int32))
    state = bd.new_model_state(w, 2, tokens.device)
    announce("state record roundtrip")
    bd.model_forward_logits(tokens[:, :20], w, state=state)
    path = tmp_path / "state.bdh"
    bd.save_model_state(path, state)
    loaded = bd.load_model_state(path, tokens.device)
    torch.cuda.synchronize()
    assert loaded.position == state.position == 20
    for a, b in zip(loaded.rho, state.rho):
        assert torch.equal(a, b)
    # continue both for four tokens: identical logits
    for t in range(20, 24):
        la = bd.model_forward_logits(tokens[:, t:t + 1].contiguous(), w, state=state)
        lb = bd.model_forward_logits(tokens[:, t:t + 1].contiguous(), w, state=loaded)
        torch.cuda.synchronize()
        assert torch.equal(la, lb), t


def test_python_written_record_loads_and_corruption_is_caught(tmp_path):
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    rng = np.random.default_rng(32)
    r0 = rng.standard_normal((2, 2, 64, 32)).astype(np.float32)
    r2 = rng.standard_normal((2, 2, 64, 32)).astype(np.float32)
    path = tmp_path / "py.bdh"
    staterec.write_record(path, 77, [(r0, 1, 1), (None, 1, 1), (r2, 1, 1)])
    announce("state record python writer")
    st = bd.load_model_state(path, torch.device("cuda"))
    assert st.position == 77 and st.rho[1] is None
    assert np.array_equal(host(st.rho[0]), r0) and np.array_equal(host(st.rho[2]), r2)
    # a record saved by the library carries the same checksum as Python's
    out = tmp_path / "lib.bdh"
    bd.save_model_state(out, st)
    lib_bytes, py_bytes = out.read_bytes(), path.read_bytes()
    assert lib_bytes[:24 + 64 * 3] == py_bytes[:24 + 64 * 3]  # header, entries, CRC32Cs
    assert lib_bytes.rstrip(b"\0") == py_bytes.rstrip(b"\0")
    blob = bytearray(path.read_bytes())
    blob[4096 + 100] ^= 0x40  # one bit of layer 0's rho
    bad = tmp_path / "bad.bdh"
    bad.write_bytes(bytes(blob))
    with pytest.raises(_lib.BdhError, match="checksum"):
        bd.load_model_state(bad, torch.device("cuda"))


def test_failed_load_leaves_the_destination_unchanged(tmp_path):
    # A checksum failure in the last layer is found before any layer is
    # copied: the caller's rho buffers keep their contents.
    import ctypes
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(33)
    shapes = [(2, 2, 64, 32), (1, 2, 128, 16), (2, 1, 32, 64)]
    rec = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    path = tmp_path / "three.bdh"
    staterec.write_record(path, 5, [(r, 1, 0) for r in rec])
    blob = bytearray(path.read_bytes())
    blob[-16] ^= 0x01  # inside the last layer's block
    bad = tmp_path / "bad_last.bdh"
    bad.write_bytes(bytes(blob))
    descs = (_lib.BdhLayerStateDesc * 3)()
    for i, s in enumerate(shapes):
        descs[i].batch, descs[i].heads, descs[i].latent, descs[i].embd = s
        descs[i].persist_sequence_state, descs[i].retain_terminal_sequence_state = 1, 0
    live = [dev(torch, rng.standard_normal(s).astype(np.float32)) for s in shapes]
    before = [t.clone() for t in live]
    ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in live])
    announce("state record failed load")
    st = lib.bdh_state_record_load(str(bad).encode(), 3, descs, ptrs, None)
    torch.cuda.synchronize()
    assert st == _lib.BDH_EINVAL and "checksum" in _lib.last_error()
    for a, b in zip(live, before):
        assert torch.equal(a, b)
    # the intact record loads into the same buffers
    assert lib.bdh_state_record_load(str(path).encode(), 3, descs, ptrs, None) == _lib.BDH_OK
    torch.cuda.synchronize()
    for t, r in zip(live, rec):
        assert np.array_equal(host(t), r)
