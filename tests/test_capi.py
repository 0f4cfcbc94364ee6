"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/volta_hip.h declares, and its host logic (algorithm selection, error
statuses) behaves as the reference's does.  No kernel is launched here."""
import ctypes

import pytest
import torch

import oracle
import volta_amd
from volta_amd import _lib, ops


def test_library_loads_and_exports_every_header_symbol():
    lib = volta_amd.lib()
    declared = _lib.header_symbols()
    assert len(declared) >= 29
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(declared) == sorted(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_auto_select_matches_reference_rule():
    # vh_conv_algo_auto_select restates conv.rs:29-69; the oracle is pinned in test_oracle.py
    for B in (1, 2, 4, 5, 64, 128):
        for C in (1, 3, 32, 64):
            for H in (3, 8, 14, 28, 56):
                for K in (1, 3, 5):
                    for gpu in (0, 1):
                        a = volta_amd.lib().vh_conv_algo_auto_select(B, C, H, H, K, gpu)
                        assert a == oracle.auto_select(B, C, H, H, K, gpu), (B, C, H, K, gpu)


def test_mi355x_selector():
    sel = volta_amd.lib().vh_conv_algo_select_mi355x
    assert sel(64, 1, 32, 28, 28, 3, 3, 1, 1, 1, 1) == volta_amd.ALGO_DIRECT  # C*K*K = 9
    assert sel(64, 32, 64, 28, 28, 3, 3, 1, 1, 1, 1) == volta_amd.ALGO_IGEMM
    assert sel(128, 64, 128, 56, 56, 1, 1, 2, 2, 0, 0) == volta_amd.ALGO_IGEMM


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device status")
def test_no_device_status_and_none_fallback():
    lib = volta_amd.lib()
    assert lib.vh_init() == _lib.VH_ERR_NO_DEVICE
    assert lib.vh_matmul(0, None, None, None, 2, 2, 2, None) == _lib.VH_ERR_NO_DEVICE
    assert b"no HIP device" in lib.vh_last_error()
    # gpu_* return None on CPU storage, like the reference's Option::None
    a = torch.ones(2, 2)
    assert ops.gpu_matmul(a, a, 2, 2, 2) is None
    with pytest.raises(volta_amd.VoltaHipError):
        volta_amd.check(lib.vh_stream_sync(None))


def test_pixel_shuffle_rejects_bad_channels():
    ps = volta_amd.PixelShuffle(3)
    with pytest.raises(ValueError):
        ps.forward(torch.empty(1, 10, 2, 2))
    with pytest.raises(ValueError):
        volta_amd.PixelShuffle(0)


def test_size_mismatch_raises_before_any_launch():
    # The C ABI carries no tensor sizes; the wrappers compare each tensor with its
    # dimensions and raise VH_ERR_BAD_SHAPE first (checked here on host tensors).
    with pytest.raises(volta_amd.VoltaHipError) as e:
        ops.expect_numel(torch.empty(5), 6, "x")
    assert e.value.status == _lib.VH_ERR_BAD_SHAPE
    ops.expect_numel(torch.empty(2, 3), 6, "x")
    ops.expect_numel(None, 6, "absent output")
    sizes = ops._CONV_OPERANDS
    assert set(sizes) == {"vh_direct_conv", "vh_igemm", "vh_conv_backward_input", "vh_igemm_backward_input",
                          "vh_conv_backward_weight", "vh_igemm_backward_weight"}
