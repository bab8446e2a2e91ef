"""The hot path under HIP graph capture: launch-bound callers (a solver's step loop, a serving
loop) capture a sequence of transforms once and replay it. Each op here is captured in a
torch.cuda.CUDAGraph after an eager warm-up (which builds the per-device caches: twiddle table,
occupancy queries), then replayed three times on new inputs copied into the captured input
tensor, with eager calls of the same op in between; every replay must equal the eager result bit
for bit (same kernels, same inputs). The ops here allocate nothing of their own: their outputs
and workspaces come from torch, which gives a captured graph its own memory pool."""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import spectral
from oracle.tolerance import random_complex, random_real
from spectral.flow import Flow
from spectral.flow.gpu import GpuSolver

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parents[1] / "gpu-spectral-stack_amd" / "python" / "spectral" \
    / "libspectral_hip.so"
STOCKHAM_R8 = 3


def replay_matches_eager(fn, inputs):
    """fn(x) -> tensor; inputs: list of same-shape device tensors (the first used for capture)."""
    static = inputs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn(static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn(static)
    for x in inputs[1:] + inputs[:1]:
        static.copy_(x)
        graph.replay()
        eager = fn(x)  # eager work between replays, on the same stream
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def cuda(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


@pytest.mark.parametrize("impl", ["stockham_r4", "stockham_r8", "stockham_r8_table"])
def test_c2c_forward_and_inverse_under_capture(rng, impl):
    inputs = [cuda(random_complex(rng, (64, 1024))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.fft_c2c(spectral.fft_c2c(x, impl=impl), inverse=True, impl=impl),
        inputs)


@pytest.mark.parametrize("n", [1024, 8192, 16384])
def test_c2c_single_pass_sizes_under_capture(rng, n):
    inputs = [cuda(random_complex(rng, (8, n))) for _ in range(3)]
    replay_matches_eager(lambda x: spectral.fft_c2c(x, impl="stockham_r8"), inputs)


def test_real_transforms_under_capture(rng):
    inputs = [cuda(random_real(rng, (256, 1024))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.irfft(spectral.rfft(x, impl="stockham_r8"), 1024, impl="stockham_r8"),
        inputs)


@pytest.mark.parametrize(("n", "arrays"), [(128, 16), (512, 2)])
def test_rfft2_and_irfft2_under_capture(rng, n, arrays):
    # 128^2 runs the single-pass kernels, 512^2 the column pass and the row-pair pass with a
    # workspace between them.
    inputs = [cuda(random_real(rng, (arrays, n, n))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.irfft2(spectral.rfft2(x, impl="stockham_r8"), n, impl="stockham_r8"),
        inputs)


@pytest.mark.parametrize(("shape", "arrays"), [((128, 128), 12), ((64, 128), 6)])
def test_persistent_complex_fft2_under_capture(rng, shape, arrays):
    # Persistent kernels: each workgroup loops over arrays g, g + G, ... with G the workgroups
    # that fit at once (an occupancy query made on the eager warm-up and cached per kernel).
    inputs = [cuda(random_complex(rng, (arrays, *shape))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.fft2(spectral.fft2(x, impl="stockham_r8"), inverse=True,
                                impl="stockham_r8"),
        inputs)


def test_transpose_method_512_under_capture(rng):
    # The inverse's transposed-side pass at 512 points is a persistent tile loop.
    inputs = [cuda(random_real(rng, (2, 512, 512))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.irfft2(spectral.rfft2(x, impl="stockham_r8", columns="transpose"),
                                  512, impl="stockham_r8", columns="transpose"),
        inputs)


def test_fno_modes_under_capture(rng):
    inputs = [cuda(random_real(rng, (2, 8, 128, 128))) for _ in range(3)]
    replay_matches_eager(
        lambda x: spectral.irfft2_from_modes(
            spectral.rfft2_truncated(x, 16, 16, impl="stockham_r8"), (128, 128),
            impl="stockham_r8"),
        inputs)


def test_fused_navier_stokes_steps_under_capture(rng):
    n = 128
    solver = GpuSolver(n, Flow(viscosity=2e-3), 0.0025, fft_impl="stockham_r8", pruned=True)
    assert solver.fused
    fields = [solver.to_spectral(cuda(random_real(rng, (4, n, n)))) for _ in range(3)]

    def steps(w_hat):
        for _ in range(4):
            w_hat = solver.step(w_hat)
        return w_hat

    replay_matches_eager(steps, fields)


@pytest.mark.parametrize("n", [64, 128])
def test_navier_stokes_many_step_launch_under_capture(rng, n):
    solver = GpuSolver(n, Flow(viscosity=np.array([1e-3, 3e-3, 5e-3])), 0.0025,
                       fft_impl="stockham_r8", pruned=True)
    fields = [solver.to_spectral(cuda(random_real(rng, (3, n, n)))) for _ in range(3)]
    replay_matches_eager(lambda w_hat: solver.advance(w_hat, 6), fields)


@pytest.mark.parametrize(("n", "batch"), [(1 << 20, 2), (1 << 22, 1)])
def test_large_c2c_without_allocation_under_capture(rng, n, batch):
    # Beyond 16384 points spx_c2c takes stream-ordered scratch; spx_c2c_noalloc, the entry point
    # for callers that cannot allocate, uses the library's static array, so the two- and
    # three-pass transforms can be captured.
    lib = ctypes.CDLL(str(LIB))
    lib.spx_last_error.restype = ctypes.c_char_p

    def fn(x):
        y = torch.empty_like(x)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.spx_c2c_noalloc(STOCKHAM_R8, ctypes.c_void_p(x.data_ptr()),
                                 ctypes.c_void_p(y.data_ptr()), n, batch, 0, stream)
        assert rc == 0, lib.spx_last_error().decode()
        return y

    inputs = [cuda(random_complex(rng, (batch, n))) for _ in range(3)]
    replay_matches_eager(fn, inputs)
