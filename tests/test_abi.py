"""CPU checks of the drop-in boundary: libbdh_hip.so loads and exports every
function include/bdh_hip.h declares, the ctypes signatures cover exactly that
set, and the Python surface returns None (the reference's fallback signal)
when no supported device is present.  No kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bdh_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(bdh_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_expected_surface():
    names = declared_functions()
    for required in ("bdh_recurrent_plan_new", "bdh_supports_backend",
                     "bdh_recurrent_attention_fwd", "bdh_recurrent_attention_rope_fwd",
                     "bdh_decode_step", "bdh_dense_causal_attention_fwd", "bdh_profile_reset",
                     "bdh_profile_get", "bdh_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from burn_dragon_amd import _lib
    lib = _lib.load()
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(raw, name), f"{name} not exported"
    assert set(_lib.SIGNATURES) == set(declared_functions())
    assert lib.bdh_version().decode().startswith("bdh_hip")


def test_plan_validation_matches_reference_none_cases():
    # recurrent.rs:187-195: zero dims and value_heads not in {1, H} -> None.
    from burn_dragon_amd import _lib
    lib = _lib.load()
    p = _lib.BdhRecurrentPlan()
    assert lib.bdh_recurrent_plan_new(2, 4, 1, 8, 16, 8, ctypes.byref(p)) == _lib.BDH_OK
    assert (p.batch, p.heads, p.value_heads, p.time, p.latent, p.embd) == (2, 4, 1, 8, 16, 8)
    assert lib.bdh_recurrent_plan_new(2, 4, 4, 8, 16, 8, ctypes.byref(p)) == _lib.BDH_OK
    assert lib.bdh_recurrent_plan_new(2, 4, 2, 8, 16, 8, ctypes.byref(p)) == _lib.BDH_UNSUPPORTED
    for dims in ((0, 4, 1, 8, 16, 8), (2, 0, 1, 8, 16, 8), (2, 4, 1, 0, 16, 8),
                 (2, 4, 1, 8, 0, 8), (2, 4, 1, 8, 16, 0)):
        assert lib.bdh_recurrent_plan_new(*dims, ctypes.byref(p)) == _lib.BDH_UNSUPPORTED
    assert "zero" in _lib.last_error()
    assert lib.bdh_recurrent_plan_new(2, 4, 1, 8, 16, 8, None) == _lib.BDH_EINVAL


def test_profile_counters_reset_and_read():
    from burn_dragon_amd import recurrent_profile_reset, recurrent_profile_snapshot
    recurrent_profile_reset()
    snap = recurrent_profile_snapshot()
    assert snap.calls == 0 and snap.launches == 0 and snap.total_ns == 0


def test_python_surface_returns_none_without_device():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: covered by the gpu tests")
    import burn_dragon_amd as bd
    q = torch.zeros(1, 2, 4, 8)
    v = torch.zeros(1, 1, 4, 8)
    assert bd.supports_recurrent_backend() is False
    assert bd.try_fused_recurrent_attention(q, v) is None
    assert bd.try_fused_dense_causal_attention(q, v, torch.ones(2)) is None
    assert bd.decode_step(q[:, :, 0], v[:, :, 0], torch.zeros(1, 2, 8, 8)) is None


def test_forward_rejects_misaligned_pointers_before_any_launch():
    # Argument checks run before any device call, so fake addresses are safe.
    from burn_dragon_amd import _lib
    lib = _lib.load()
    p = _lib.BdhRecurrentPlan()
    assert lib.bdh_recurrent_plan_new(1, 2, 1, 8, 16, 8, ctypes.byref(p)) == _lib.BDH_OK
    good, bad = 0x10000, 0x10008
    for q, v, ctx, rho in ((bad, good, good, good), (good, bad, good, good),
                           (good, good, bad, good), (good, good, good, bad)):
        st = lib.bdh_recurrent_attention_fwd(ctypes.byref(p), _lib.BDH_F32, q, v, None, None,
                                             ctx, rho, 0, None)
        assert st == _lib.BDH_EINVAL
        assert "aligned" in _lib.last_error()


def test_decode_step_rejects_misaligned_pointers_before_any_launch():
    # The one-token step reads fp32 rows: every pointer must be 4-byte aligned.
    from burn_dragon_amd import _lib
    lib = _lib.load()
    good, bad = 0x10000, 0x10002
    for x, v, rho, a in ((bad, good, good, good), (good, bad, good, good),
                         (good, good, bad, good), (good, good, good, bad)):
        st = lib.bdh_decode_step(1, 2, 1, 16, 8, x, v, rho, None, None, a, None, None, None)
        assert st == _lib.BDH_EINVAL
        assert "aligned" in _lib.last_error()
