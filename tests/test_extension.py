"""The PyTorch extension (reference tests/test_extension.py): operators registered, registry
names from the library, our kernel runs on PyTorch's current stream, the dispatcher refuses CPU
tensors, bad dtypes are refused."""

import pytest
import torch

import spectral


def test_operators_are_registered():
    for name in ["scale", "fft_c2c", "fft_r2c", "fft_c2r", "fft2_c2c", "fft2_r2c", "fft2_c2r",
                 "fft_c2c_pruned", "rfft2_modes", "irfft2_modes"]:
        assert hasattr(torch.ops.spectral, name)


def test_schema_matches_the_reference():
    s = str(torch.ops.spectral.fft2_r2c.default._schema)
    assert s == 'spectral::fft2_r2c(Tensor x, str impl="naive", str columns="auto") -> Tensor'
    s = str(torch.ops.spectral.fft_c2c_pruned.default._schema)
    assert "int keep, bool inverse=False" in s


def test_fft_implementations_come_from_the_registry():
    assert spectral.FFT_IMPLS[0] == "naive"
    assert spectral.FFT_IMPLS == ("naive", "stockham_r2", "stockham_r4", "stockham_r8",
                                  "stockham_r8_table")


def test_cpu_input_is_rejected_by_the_dispatcher():
    x = torch.zeros(4, dtype=torch.complex64)
    with pytest.raises(NotImplementedError, match="CPU"):
        spectral.scale(x, 0.5)
    with pytest.raises(NotImplementedError, match="CPU"):
        spectral.fft_c2c(torch.zeros(2, 8, dtype=torch.complex64), impl="stockham_r8")


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 255, 256, 257, 2047, 2048, 2049, 4096 * 3 + 2, 1 << 20,
                               (1 << 20) + 1])
def test_scale_matches_torch(n):
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(n, dtype=torch.complex64, device="cuda", generator=g)
    # multiplying by 0.5 is exact: bit-for-bit equality
    torch.testing.assert_close(spectral.scale(x, 0.5), x * 0.5, rtol=0, atol=0)


@pytest.mark.gpu
def test_scale_non_contiguous_and_misaligned_input():
    x = torch.randn(1001, dtype=torch.complex64, device="cuda")
    torch.testing.assert_close(spectral.scale(x[::2], 0.5), x[::2] * 0.5, rtol=0, atol=0)
    torch.testing.assert_close(spectral.scale(x[1:], 0.5), x[1:] * 0.5, rtol=0, atol=0)


@pytest.mark.gpu
def test_scale_on_a_side_stream():
    x = torch.randn(1 << 20, dtype=torch.complex64, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y = spectral.scale(x, 0.5)
    side.synchronize()
    torch.testing.assert_close(y, x * 0.5, rtol=0, atol=0)


@pytest.mark.gpu
def test_wrong_dtype_is_rejected():
    x = torch.zeros(4, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="complex64"):
        spectral.scale(x, 0.5)
