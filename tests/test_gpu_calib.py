"""The HBM calibration kernels behind ``bench.py --only rmw`` do the work
they are credited with: the copy copies, the in-place RMW adds (1, 0, 0, 0)
to every 16-byte group, the row RMW adds it to exactly the listed 1 KiB rows
(indices outside the buffer skipped), and the read leaves its sink alone."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu


def test_calibration_kernels_do_the_credited_work():
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    nbytes = 1 << 20
    rows_total = nbytes // 1024
    rng = np.random.default_rng(5)
    base = torch.from_numpy(rng.standard_normal(nbytes // 4).astype(np.float32)).cuda()
    a, b = base.clone(), torch.zeros_like(base)
    sink = torch.zeros(4, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    announce("calib hbm", nbytes)
    assert lib.bdh_calib_hbm(_lib.BDH_CALIB_READ, p(a), p(sink), nbytes, None, 0, stream) == _lib.BDH_OK
    assert lib.bdh_calib_hbm(_lib.BDH_CALIB_COPY, p(a), p(b), nbytes, None, 0, stream) == _lib.BDH_OK
    torch.cuda.synchronize()
    assert torch.equal(b, base) and torch.equal(sink, torch.zeros_like(sink))
    assert lib.bdh_calib_hbm(_lib.BDH_CALIB_RMW, p(a), None, nbytes, None, 0, stream) == _lib.BDH_OK
    torch.cuda.synchronize()
    want = base.clone().view(-1, 4)
    want[:, 0] += 1.0
    assert torch.equal(a.view(-1, 4), want)
    pick = np.sort(rng.choice(rows_total, rows_total // 10, replace=False)).astype(np.int32)
    listed = np.concatenate([pick, np.array([-1, rows_total, 1 << 30], np.int32)])
    rows = torch.from_numpy(listed).cuda()
    a = base.clone()
    assert lib.bdh_calib_hbm(_lib.BDH_CALIB_RMW_ROWS, p(a), None, nbytes, p(rows), listed.size,
                             stream) == _lib.BDH_OK
    torch.cuda.synchronize()
    want = base.clone().view(rows_total, 64, 4)
    want[torch.from_numpy(pick.astype(np.int64)).cuda(), :, 0] += 1.0
    assert torch.equal(a.view(rows_total, 64, 4), want)
    assert lib.bdh_calib_hbm(_lib.BDH_CALIB_RMW, p(a), None, 1000, None, 0, stream) == _lib.BDH_EINVAL
    assert lib.bdh_calib_hbm(7, p(a), None, nbytes, None, 0, stream) == _lib.BDH_EINVAL


def test_mfma_calibration_reports_its_flop():
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    sink = torch.zeros(4, device="cuda")
    flop = ctypes.c_double()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    announce("calib mfma")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for kind, per_mfma, per_round in ((_lib.BDH_CALIB_MFMA_16X16X32_BF16, 2 * 16 * 16 * 32, 8),
                                      (_lib.BDH_CALIB_MFMA_32X32X16_BF16, 2 * 32 * 32 * 16, 4),
                                      (_lib.BDH_CALIB_MFMA_32X32X2_F32, 2 * 32 * 32 * 2, 4)):
        assert lib.bdh_calib_mfma(kind, 100, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(flop),
                                  stream) == _lib.BDH_OK
        torch.cuda.synchronize()
        # two 4-wave workgroups per CU, `per_round` MFMAs a round, 100 rounds
        assert flop.value == 2 * cus * 4 * 100 * per_round * per_mfma
        assert torch.equal(sink, torch.zeros_like(sink))
    assert lib.bdh_calib_mfma(5, 100, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(flop),
                              stream) == _lib.BDH_EINVAL
    assert lib.bdh_calib_mfma(0, 0, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(flop),
                              stream) == _lib.BDH_EINVAL
