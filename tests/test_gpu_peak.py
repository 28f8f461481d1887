"""GPU checks of the attained-peak microkernels behind bench.py's roofline:
the copy kernel copies exactly, and the MFMA loop reports the flops it ran."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_peak_copy_is_exact():
    from parrot import _abi
    lib = _abi.load()
    src = torch.randint(0, 255, (3 << 20,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros_like(src)
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib.parrot_peak_copy(src.data_ptr(), dst.data_ptr(), src.numel(), 512, stream),
               "parrot_peak_copy")
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    assert lib.parrot_peak_copy(src.data_ptr(), dst.data_ptr(), 17, 512, stream) == -2


@pytest.mark.parametrize("wide", [0, 1])
def test_peak_mfma_counts_its_flops(wide):
    from parrot import _abi
    lib = _abi.load()
    blocks, iters = 64, 10
    out = torch.empty(blocks * 256, device="cuda")
    flops = ctypes.c_int64()
    _abi.check(lib.parrot_peak_mfma_bf16(wide, blocks, iters, out.data_ptr(), ctypes.byref(flops),
                                         torch.cuda.current_stream().cuda_stream),
               "parrot_peak_mfma_bf16")
    torch.cuda.synchronize()
    # 4 wavefronts x chains x iters x flops per MFMA (16x16x32: 8 chains, 32x32x16: 4 chains)
    per_block = 4 * (4 * 2 * 32 * 32 * 16 if wide else 8 * 2 * 16 * 16 * 32) * iters
    assert flops.value == blocks * per_block
    assert torch.isfinite(out).all()
