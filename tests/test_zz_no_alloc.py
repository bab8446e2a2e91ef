"""spx_c2c_noalloc, the c2c entry point that allocates nothing, against spx_c2c through the C ABI:
the same kernels, so the same bits, with the large transforms' scratch in the library's static
per-device array instead of stream-ordered allocations. Calls run back to back on one GPU, so
each reuses the array the previous one left behind."""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as ref
from oracle.tolerance import assert_transform_close, random_complex

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "gpu-spectral-stack_amd" / "python" / "spectral" \
    / "libspectral_hip.so"
STOCKHAM_R8 = 3
SCRATCH_VALUES = 1 << 22


@pytest.fixture(scope="module")
def lib():
    so = ctypes.CDLL(str(LIB))
    so.spx_last_error.restype = ctypes.c_char_p
    return so


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _both(lib, x: torch.Tensor, n: int, batch: int, inverse: int):
    y_alloc = torch.full_like(x, float("nan"))
    y_static = torch.full_like(x, float("nan"))
    assert lib.spx_c2c(STOCKHAM_R8, _ptr(x), _ptr(y_alloc), n, batch, inverse, None) == 0, \
        lib.spx_last_error().decode()
    assert lib.spx_c2c_noalloc(STOCKHAM_R8, _ptr(x), _ptr(y_static), n, batch, inverse,
                               None) == 0, lib.spx_last_error().decode()
    torch.cuda.synchronize()
    return y_alloc, y_static


def test_noalloc_matches_c2c_on_calls_in_a_row(lib, rng):
    # The three-pass path filling the whole static array, then the two-pass path filling it again,
    # then a smaller two-pass call and a single-pass size that needs no scratch: each must equal
    # spx_c2c bit for bit, whatever the array held from the call before.
    for n, batch in [(1 << 22, 1), (1 << 20, 4), (1 << 17, 3), (1024, 64)]:
        assert n * batch <= SCRATCH_VALUES
        x_host = random_complex(rng, (batch, n))
        x = torch.from_numpy(x_host).cuda()
        for inverse in (0, 1):
            y_alloc, y_static = _both(lib, x, n, batch, inverse)
            assert torch.equal(y_static, y_alloc), (n, batch, inverse)
        forward = _both(lib, x, n, batch, 0)[1]
        assert_transform_close(forward.cpu().numpy()[:1], ref.fft(x_host[:1]), n)


def _hip_runtime() -> ctypes.CDLL:
    # The HIP runtime this process already mapped: the one the library and PyTorch call.
    for line in Path("/proc/self/maps").read_text().splitlines():
        if "libamdhip64.so" in line.split()[-1]:
            return ctypes.CDLL(line.split()[-1])
    return ctypes.CDLL("libamdhip64.so")


USED_MEM_HIGH = 8  # hipMemPoolAttrUsedMemHigh


def test_noalloc_takes_nothing_from_the_stream_ordered_pool(lib, rng):
    # spx_c2c's large transforms take their scratch from the device's default pool in stream
    # order (hipMallocAsync, which is also legal under graph capture), so a noalloc that fell
    # back to it would still match spx_c2c bit for bit. The pool's high-water mark of memory in
    # use tells them apart: reset to zero, it must stay zero across noalloc calls and rise for
    # the same transforms through spx_c2c.
    hip = _hip_runtime()
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), torch.cuda.current_device()) == 0
    high = ctypes.c_uint64()

    def reset_and_run(entry, cases):
        zero = ctypes.c_uint64(0)
        torch.cuda.synchronize()
        assert hip.hipMemPoolSetAttribute(pool, USED_MEM_HIGH, ctypes.byref(zero)) == 0
        for x, y, n, batch in cases:
            assert entry(STOCKHAM_R8, _ptr(x), _ptr(y), n, batch, 0, None) == 0, \
                lib.spx_last_error().decode()
        torch.cuda.synchronize()
        assert hip.hipMemPoolGetAttribute(pool, USED_MEM_HIGH, ctypes.byref(high)) == 0
        return high.value

    cases = []
    for n, batch in [(1 << 22, 1), (1 << 20, 4)]:
        x = torch.from_numpy(random_complex(rng, (batch, n))).cuda()
        cases.append((x, torch.empty_like(x), n, batch))
    assert reset_and_run(lib.spx_c2c_noalloc, cases) == 0
    assert reset_and_run(lib.spx_c2c, cases) >= (1 << 22) * 8  # the control does use the pool
    assert reset_and_run(lib.spx_c2c_noalloc, cases) == 0
