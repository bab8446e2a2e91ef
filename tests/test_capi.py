"""The C ABI of libspectral_hip.so (include/spectral_hip.h): the library loads, exports every
declared symbol, reports the registry, and rejects bad arguments with SPX_EINVAL and the
reference's messages before touching the GPU. On a GPU, direct calls match the oracle."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch  # noqa: F401  # the HIP runtime PyTorch ships must be loaded first

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "spectral_hip.h"
LIB = REPO / "gpu-spectral-stack_amd" / "python" / "spectral" / "libspectral_hip.so"
SPX_OK, SPX_EINVAL, SPX_ERUNTIME = 0, 1, 2


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(spx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    so = ctypes.CDLL(str(LIB))
    so.spx_impl_name.restype = ctypes.c_char_p
    so.spx_impl_names.restype = ctypes.c_char_p
    so.spx_last_error.restype = ctypes.c_char_p
    so.spx_impl_find.argtypes = [ctypes.c_char_p]
    return so


def test_header_declares_the_boundary():
    names = declared_functions()
    assert len(names) >= 30
    for required in ["spx_c2c", "spx_r2c", "spx_c2r", "spx_columns", "spx_fft2_r2c",
                     "spx_rfft2_modes", "spx_irfft2_modes", "spx_last_error"]:
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing


class Info(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("has_columns", ctypes.c_int),
                ("has_pruned", ctypes.c_int), ("max_n", ctypes.c_int),
                ("max_c2c_n", ctypes.c_int), ("max_real_n", ctypes.c_int),
                ("real_needs_work", ctypes.c_int), ("lazy_table", ctypes.c_int)]


def test_registry_rows(lib):
    names = [lib.spx_impl_name(i).decode() for i in range(lib.spx_impl_count())]
    assert names == ["naive", "stockham_r2", "stockham_r4", "stockham_r8", "stockham_r8_table"]
    assert lib.spx_impl_names().decode() == ", ".join(names)
    assert lib.spx_impl_find(b"stockham_r8") == 3
    assert lib.spx_impl_find(b"nope") == -1
    assert lib.spx_impl_name(99) is None
    info = Info()
    assert lib.spx_impl_get_info(0, ctypes.byref(info)) == SPX_OK
    assert (info.name, info.has_columns, info.has_pruned, info.real_needs_work) == (
        b"naive", 0, 0, 1)
    assert info.max_n == info.max_c2c_n == info.max_real_n == 1 << 30
    assert lib.spx_impl_get_info(3, ctypes.byref(info)) == SPX_OK
    assert (info.has_columns, info.has_pruned, info.max_n, info.max_c2c_n, info.max_real_n,
            info.real_needs_work) == (1, 1, 4096, 1 << 24, 8192, 0)
    tables = []
    for i in range(lib.spx_impl_count()):
        assert lib.spx_impl_get_info(i, ctypes.byref(info)) == SPX_OK
        tables.append(info.lazy_table)
    assert tables == [0, 0, 0, 0, 1]  # only stockham_r8_table builds a table on first use
    assert lib.spx_impl_get_info(9, ctypes.byref(info)) == SPX_EINVAL


def _last(lib) -> str:
    return lib.spx_last_error().decode()


def test_argument_errors_come_back_as_einval(lib):
    # Validation runs before anything is queued, so these need no GPU.
    p = ctypes.c_void_p(0x1000)
    q = ctypes.c_void_p(0x100000)
    assert lib.spx_c2c(99, p, q, 8, 1, 0, None) == SPX_EINVAL
    assert "unknown FFT implementation" in _last(lib)
    assert lib.spx_c2c(3, p, q, 12, 1, 0, None) == SPX_EINVAL
    assert "power of two" in _last(lib)
    assert lib.spx_c2c(3, p, p, 8, 1, 0, None) == SPX_EINVAL
    assert "must not overlap" in _last(lib)
    assert lib.spx_r2c(3, p, q, 16384, 1, None, None) == SPX_EINVAL
    assert "n must be a power of two from 2 to 8192" in _last(lib)
    assert lib.spx_r2c(0, p, q, 16, 1, None, None) == SPX_EINVAL
    assert "needs a workspace" in _last(lib)
    assert lib.spx_fft2_c2c(3, 1, p, q, 8192, 2, 1, 0, None, None) == SPX_EINVAL
    assert "n1 to be a power of two up to 4096" in _last(lib)
    assert lib.spx_fft2_c2c(0, 1, p, q, 8, 8, 1, 0, None, None) == SPX_EINVAL
    assert "no strided column kernel" in _last(lib)
    assert lib.spx_rfft2_modes(3, p, q, 8, 8, 5, 2, 1, None, None) == SPX_EINVAL
    assert "1 <= m1 <= n1/2" in _last(lib)
    assert lib.spx_pruned_columns(3, p, p, 8, 4, 1, 2, 0, 0, None) == SPX_EINVAL
    assert "cannot run in place" in _last(lib)
    assert lib.spx_pruned_c2c(0, p, q, 8, 1, 4, 0, None) == SPX_EINVAL
    assert "no pruned kernels" in _last(lib)


def test_navier_stokes_stage_arguments(lib):
    assert [lib.spx_ns_supports(n) for n in (32, 64, 128, 256)] == [0, 1, 1, 0]
    p = ctypes.c_void_p(0x1000)
    f = ctypes.c_float
    assert lib.spx_ns_stage(p, None, None, p, p, p, p, 0, f(0.1), f(1e-3), 32, 1, 0,
                            None) == SPX_EINVAL
    assert "supports n = 64 and 128" in _last(lib)
    assert lib.spx_ns_stage(p, None, None, p, p, p, p, 0, f(0.1), f(1e-3), 64, 1, 2,
                            None) == SPX_EINVAL
    assert "stage 0 or 1" in _last(lib)
    assert lib.spx_ns_stage(p, None, None, p, p, p, p, 0, f(0.1), f(1e-3), 64, 0, 0,
                            None) == SPX_EINVAL
    assert lib.spx_ns_stage(p, None, None, None, p, p, p, 0, f(0.1), f(1e-3), 64, 1, 0,
                            None) == SPX_EINVAL
    assert "writes both" in _last(lib)
    assert lib.spx_ns_stage(p, None, None, None, p, p, p, 0, f(0.1), f(1e-3), 64, 1, 1,
                            None) == SPX_EINVAL
    assert "stage 1 reads" in _last(lib)


def test_navier_stokes_steps_arguments(lib):
    # Rejected before anything reaches the device; steps = 0 in place is accepted and queues
    # nothing.
    state, work = 0x100000, 0x200000
    p, f = ctypes.c_void_p(0x1000), ctypes.c_float
    field = 2 * 22 * 22 * 8  # bytes of one 64^2 field's modes
    v = ctypes.c_void_p

    def steps(n=64, batch=1, count=1, nu_stride=0, w_in=state, w_out=state, wk=work):
        return lib.spx_ns_steps(v(w_in), v(w_out), v(wk), p, p, nu_stride, f(0.1), f(1e-3), n,
                                batch, count, None)

    assert steps(n=32) == SPX_EINVAL and "supports n = 64 and 128" in _last(lib)
    assert steps(batch=0) == SPX_EINVAL and "batch >= 1" in _last(lib)
    assert steps(count=-1) == SPX_EINVAL and "steps >= 0" in _last(lib)
    assert steps(nu_stride=2) == SPX_EINVAL and "nu_stride 0 or 1" in _last(lib)
    assert steps(wk=None) == SPX_EINVAL and "must not be null" in _last(lib)
    assert steps(w_out=None) == SPX_EINVAL and "must not be null" in _last(lib)
    assert steps(wk=state) == SPX_EINVAL and "must not overlap" in _last(lib)
    # The work area's end reaching into the state, the state's end into the work area, and the
    # work area over a separate output.
    assert steps(wk=state - 2 * field + 8) == SPX_EINVAL
    assert steps(wk=state + field - 8) == SPX_EINVAL
    assert steps(w_out=work + 8) == SPX_EINVAL and "overlap w_in or w_out" in _last(lib)
    # Input and output: the same array, or apart; a partial overlap is refused.
    assert steps(w_out=state + 8) == SPX_EINVAL and "the same array" in _last(lib)
    assert steps(wk=state - 2 * field, count=0) == SPX_OK
    assert steps(wk=state + field, count=0) == SPX_OK


def test_workspace_queries(lib):
    count = ctypes.c_size_t()
    assert lib.spx_fft2_c2c_workspace(3, 1, 8, 8, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 0
    # The transpose method: the Stockham implementations' two passes go through one array-sized
    # region (n2 x n1, or (n2/2 + 1) x n1 for real transforms); naive's four kernels through two,
    # plus its real-row scratch; a side of 1, real rows of 2 and complex arrays with a side
    # beyond 1024 take the four-kernel route too.
    assert lib.spx_fft2_c2c_workspace(3, 0, 8, 8, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 8 * 8 * 2
    assert lib.spx_fft2_r2c_workspace(3, 0, 8, 8, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 8 * 5 * 2
    assert lib.spx_fft2_c2r_workspace(1, 0, 16, 32, 3, ctypes.byref(count)) == SPX_OK
    assert count.value == 16 * 17 * 3
    assert lib.spx_fft2_c2c_workspace(3, 0, 1, 8, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 2 * 1 * 8 * 2
    assert lib.spx_fft2_r2c_workspace(4, 0, 8, 2, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 2 * 8 * 2 * 2
    assert lib.spx_fft2_r2c_workspace(0, 0, 8, 8, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 2 * 8 * 5 * 2 + 8 * 4 * 2
    assert lib.spx_fft2_c2c_workspace(3, 0, 1024, 16, 1, ctypes.byref(count)) == SPX_OK
    assert count.value == 1024 * 16
    assert lib.spx_fft2_c2c_workspace(3, 0, 2048, 16, 1, ctypes.byref(count)) == SPX_OK
    assert count.value == 2 * 2048 * 16
    assert lib.spx_fft2_r2c_workspace(3, 0, 2048, 2048, 1, ctypes.byref(count)) == SPX_OK
    assert count.value == 2048 * 1025
    # 128 x 128 runs as one single-pass kernel (no workspace); 512 x 512 as rows then columns,
    # through n1 x m2 values per array.
    assert lib.spx_rfft2_modes_workspace(3, 128, 128, 16, 16, 4, ctypes.byref(count)) == SPX_OK
    assert count.value == 0
    assert lib.spx_rfft2_modes_workspace(3, 512, 512, 16, 16, 4, ctypes.byref(count)) == SPX_OK
    assert count.value == 512 * 16 * 4
    assert lib.spx_fft2_r2c_workspace(3, 1, 128, 128, 2, ctypes.byref(count)) == SPX_OK
    assert count.value == 0
    assert lib.spx_fft_c2c_pruned_workspace(0, 64, 8, 3, ctypes.byref(count)) == SPX_OK
    assert count.value == 64 * 3
    # naive: the real rows' n1 x w, the m2 kept columns' m2 x n1, and its real-row scratch
    assert lib.spx_rfft2_modes_workspace(0, 64, 32, 4, 5, 3, ctypes.byref(count)) == SPX_OK
    assert count.value == 3 * (64 * 17 + 5 * 64 + 64 * 16)
    assert lib.spx_irfft2_modes_workspace(0, 64, 32, 4, 5, 3, ctypes.byref(count)) == SPX_OK
    assert count.value == 3 * (64 * 17 + 5 * 64 + 64 * 16)


@pytest.mark.gpu
def test_direct_calls_on_an_explicit_stream(lib, rng):
    from oracle import reference as ref
    from oracle.tolerance import assert_transform_close, random_complex, random_real

    x = random_complex(rng, (64, 1024))
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    rc = lib.spx_c2c(3, ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(yd.data_ptr()), 1024, 64,
                     0, ctypes.c_void_p(stream.cuda_stream))
    assert rc == SPX_OK, _last(lib)
    stream.synchronize()
    assert_transform_close(yd, ref.fft(x), 1024)

    r = random_real(rng, (32, 2048))
    rd = torch.from_numpy(r).cuda()
    cd = torch.empty(32, 1025, dtype=torch.complex64, device="cuda")
    rc = lib.spx_r2c(3, ctypes.c_void_p(rd.data_ptr()), ctypes.c_void_p(cd.data_ptr()), 2048, 32,
                     None, ctypes.c_void_p(stream.cuda_stream))
    assert rc == SPX_OK, _last(lib)
    stream.synchronize()
    assert_transform_close(cd, ref.rfft(r), 2048)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.gpu
def test_direct_2d_and_modes_calls(lib, rng):
    # Single-pass (128 x 128), column-first (512 x 512) and pruned paths through the C ABI itself,
    # with the workspace the query asks for.
    from oracle import reference as ref
    from oracle.tolerance import assert_transform_close, random_complex, random_real

    for n in (128, 512):
        r = random_real(rng, (3, n, n))
        rd = torch.from_numpy(r).cuda()
        yd = torch.empty(3, n, n // 2 + 1, dtype=torch.complex64, device="cuda")
        count = ctypes.c_size_t()
        assert lib.spx_fft2_r2c_workspace(3, 1, n, n, 3, ctypes.byref(count)) == SPX_OK
        work = torch.empty(max(count.value, 1), dtype=torch.complex64, device="cuda")
        assert lib.spx_fft2_r2c(3, 1, _ptr(rd), _ptr(yd), n, n, 3, _ptr(work), None) == SPX_OK
        assert lib.spx_fft2_c2r_workspace(3, 1, n, n, 3, ctypes.byref(count)) == SPX_OK
        work2 = torch.empty(max(count.value, 1), dtype=torch.complex64, device="cuda")
        back = torch.empty_like(rd)
        assert lib.spx_fft2_c2r(3, 1, _ptr(yd), _ptr(back), n, n, 3, _ptr(work2), None) == SPX_OK
        torch.cuda.synchronize()
        assert_transform_close(yd, ref.rfft2(r), n * n, axes=(-2, -1))
        assert_transform_close(back, r, n * n, axes=(-2, -1))

    x = random_complex(rng, (5, 64, 64))
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    assert lib.spx_fft2_c2c(3, 1, _ptr(xd), _ptr(yd), 64, 64, 5, 0, None, None) == SPX_OK
    torch.cuda.synchronize()
    assert_transform_close(yd, ref.fft2(x), 64 * 64, axes=(-2, -1))

    r = random_real(rng, (4, 128, 128))
    rd = torch.from_numpy(r).cuda()
    md = torch.empty(4, 32, 16, dtype=torch.complex64, device="cuda")
    assert lib.spx_rfft2_modes(3, _ptr(rd), _ptr(md), 128, 128, 16, 16, 4, None, None) == SPX_OK
    out = torch.empty_like(rd)
    assert lib.spx_irfft2_modes(3, _ptr(md), _ptr(out), 128, 128, 16, 16, 4, None, None) == SPX_OK
    torch.cuda.synchronize()
    modes = ref.rfft2_truncate(r, 16, 16)
    assert_transform_close(md, modes, 128 * 128, axes=(-2, -1))
    assert_transform_close(out, ref.irfft2_from_modes(modes, (128, 128)), 128 * 128,
                           axes=(-2, -1))


@pytest.mark.gpu
def test_direct_radio_and_navier_stokes_calls(lib, rng):
    import numpy as np
    import scipy.signal

    from oracle.tolerance import random_complex, random_real
    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    ll = ctypes.c_longlong
    x = random_complex(rng, (2, 3000))
    taps = random_real(rng, 63)
    h = np.zeros(256, dtype=np.complex64)
    h[:63] = taps
    xd = torch.from_numpy(x).cuda()
    hd = torch.from_numpy(np.fft.fft(h).astype(np.complex64)).cuda()
    yd = torch.empty_like(xd)
    assert lib.spx_rf_fir(3, _ptr(xd), _ptr(hd), _ptr(yd), ll(3000), 63, 256, ll(2), None) == SPX_OK
    spec = torch.empty(2, 3, 1024, dtype=torch.complex64, device="cuda")
    assert lib.spx_rf_spectrum(3, _ptr(xd), None, _ptr(spec), ll(3000), 1024, ll(2), None) == SPX_OK
    torch.cuda.synchronize()
    expected = scipy.signal.lfilter(taps.astype(np.float64), 1.0, x.astype(np.complex128))
    assert np.linalg.norm(yd.cpu().numpy() - expected) / np.linalg.norm(expected) < 2e-5
    padded = np.zeros((2, 3072), dtype=np.complex128)
    padded[:, :3000] = x
    frames = np.fft.fft(padded.reshape(2, 3, 1024), axis=-1)
    assert np.linalg.norm(spec.cpu().numpy() - frames) / np.linalg.norm(frames) < 1e-5

    # One predictor stage of 3 fields of 64^2 against the solver's own fused operator.
    solver = GpuSolver(64, Flow(viscosity=np.array([1e-3, 2e-3, 3e-3])), 2.5e-3, pruned=True)
    w = solver.to_spectral(torch.from_numpy(rng.standard_normal((3, 64, 64))).float().cuda())
    f0 = torch.empty_like(w)
    pred = torch.empty_like(w)
    assert lib.spx_ns_stage(_ptr(w), None, None, _ptr(f0), _ptr(pred), _ptr(solver.forcing_hat),
                            ctypes.c_void_p(solver.nu.data_ptr()), 1, ctypes.c_float(0.1),
                            ctypes.c_float(2.5e-3), 64, 3, 0, None) == SPX_OK
    ref_f0, ref_pred = torch.ops.spectral.ns_predict(w, solver.forcing_hat, solver.nu, 0.1,
                                                     2.5e-3, 64)
    torch.cuda.synchronize()
    assert torch.equal(f0, ref_f0) and torch.equal(pred, ref_pred)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [64, 128])
def test_ns_stage_may_write_over_its_inputs(lib, rng, n):
    # Stage 0 with the predictor written over the state, stage 1 with the new state written over
    # w0 and then over the predictor: each must equal the same stage into fresh outputs.
    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    solver = GpuSolver(n, Flow(viscosity=np.array([1e-3, 4e-3])), 2.5e-3, pruned=True)
    w = solver.to_spectral(torch.from_numpy(rng.standard_normal((2, n, n))).float().cuda())
    args = (_ptr(solver.forcing_hat), ctypes.c_void_p(solver.nu.data_ptr()), 1,
            ctypes.c_float(0.1), ctypes.c_float(2.5e-3), n, 2)
    f0 = torch.empty_like(w)
    pred = torch.empty_like(w)
    assert lib.spx_ns_stage(_ptr(w), None, None, _ptr(f0), _ptr(pred), *args, 0, None) == SPX_OK
    new = torch.empty_like(w)
    assert lib.spx_ns_stage(_ptr(pred), _ptr(w), _ptr(f0), None, _ptr(new), *args, 1,
                            None) == SPX_OK

    over = w.clone()
    f0_over = torch.empty_like(w)
    assert lib.spx_ns_stage(_ptr(over), None, None, _ptr(f0_over), _ptr(over), *args, 0,
                            None) == SPX_OK
    w0 = w.clone()
    assert lib.spx_ns_stage(_ptr(pred), _ptr(w0), _ptr(f0), None, _ptr(w0), *args, 1,
                            None) == SPX_OK
    p = pred.clone()
    assert lib.spx_ns_stage(_ptr(p), _ptr(w), _ptr(f0), None, _ptr(p), *args, 1, None) == SPX_OK
    torch.cuda.synchronize()
    assert torch.equal(over, pred) and torch.equal(f0_over, f0)
    assert torch.equal(w0, new) and torch.equal(p, new)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [64, 128])
def test_ns_steps_equal_alternating_stages(lib, rng, n):
    # Steps in one launch against spx_ns_stage launches into fresh outputs, to float32 rounding
    # (the two kernels contract some products into fused multiply-adds differently: their
    # tendencies differ in almost every mode by a few ulps, and each is as far from the composed
    # float32 path as the other, 2-6e-6), out of place and in place, with the work area holding
    # the last step's tendency and predictor. The tendency, a difference of the forcing and the
    # nonlinear term, carries the larger relative rounding. The launch is deterministic: every
    # run from the same state gives the same bits, in place or not.
    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    solver = GpuSolver(n, Flow(viscosity=np.array([1e-3, 4e-3, 2e-3])), 2.5e-3, pruned=True)
    w = solver.to_spectral(torch.from_numpy(rng.standard_normal((3, n, n))).float().cuda())
    kept = w.clone()
    args = (_ptr(solver.forcing_hat), ctypes.c_void_p(solver.nu.data_ptr()), 1,
            ctypes.c_float(0.1), ctypes.c_float(2.5e-3), n, 3)

    def rel(a, b):
        return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))

    state, done = w, 0
    for steps, bound in ((1, 1e-6), (4, 1e-5)):  # the state's and the predictor's
        while done < steps:
            f0, pred, new = torch.empty_like(w), torch.empty_like(w), torch.empty_like(w)
            assert lib.spx_ns_stage(_ptr(state), None, None, _ptr(f0), _ptr(pred), *args, 0,
                                    None) == SPX_OK
            assert lib.spx_ns_stage(_ptr(pred), _ptr(state), _ptr(f0), None, _ptr(new), *args,
                                    1, None) == SPX_OK
            state, done = new, done + 1
        runs = []
        for in_place in (False, True, False):
            out = w.clone() if in_place else torch.full_like(w, float("nan"))
            work = torch.full((2,) + tuple(w.shape), float("nan"), dtype=w.dtype,
                              device=w.device)
            source = out if in_place else w
            assert lib.spx_ns_steps(_ptr(source), _ptr(out), _ptr(work), *args, steps,
                                    None) == SPX_OK
            runs.append((out, work))
        torch.cuda.synchronize()
        assert torch.equal(w, kept)
        (out, work) = runs[0]
        for again, work_again in runs[1:]:
            assert torch.equal(out, again) and torch.equal(work, work_again)
        assert rel(out, state) < bound, f"{steps} steps"
        assert rel(work[1], pred) < bound, f"{steps} steps"
        assert rel(work[0], f0) < 2e-5, f"{steps} steps"
    # No steps: a copy.
    out = torch.full_like(w, float("nan"))
    assert lib.spx_ns_steps(_ptr(w), _ptr(out), _ptr(work), *args, 0, None) == SPX_OK
    torch.cuda.synchronize()
    assert torch.equal(out, w)


def _fft_columns(x: np.ndarray, inverse: bool) -> np.ndarray:
    from oracle import reference as ref

    cols_last = np.swapaxes(x, -1, -2)
    return np.swapaxes(ref.ifft(cols_last) if inverse else ref.fft(cols_last), -1, -2)


@pytest.mark.gpu
@pytest.mark.parametrize(("n", "slabs"), [(256, 1040), (512, 300)])
def test_direct_columns_over_many_tiles(lib, rng, n, slabs):
    # 17 columns per slab: more tiles of 16 columns than the device holds workgroups at once, so
    # each workgroup of the persistent column kernel walks several, and the last tile is partial.
    # Out of place and in place, forward and inverse, and both pruned sides.
    from oracle.tolerance import assert_transform_close, random_complex

    cols, m1 = 17, 8
    x = random_complex(rng, (slabs, n, cols))
    xd = torch.from_numpy(x).cuda()
    for inverse in (0, 1):
        yd = torch.empty_like(xd)
        assert lib.spx_columns(3, _ptr(xd), _ptr(yd), n, cols, slabs, inverse, None) == SPX_OK
        inplace = xd.clone()
        assert lib.spx_columns(3, _ptr(inplace), _ptr(inplace), n, cols, slabs, inverse,
                               None) == SPX_OK
        torch.cuda.synchronize()
        expected = _fft_columns(x, bool(inverse))
        assert_transform_close(yd, expected, n, axes=(-2,))
        assert torch.equal(inplace, yd)

    # Forward keeping rows 0 .. m1-1 and n-m1 .. n-1; inverse from those rows alone.
    kept = torch.empty(slabs, 2 * m1, cols, dtype=torch.complex64, device="cuda")
    assert lib.spx_pruned_columns(3, _ptr(xd), _ptr(kept), n, cols, slabs, 0, m1, 0,
                                  None) == SPX_OK
    full = _fft_columns(x, False)
    rows = np.r_[0:m1, n - m1:n]
    modes = random_complex(rng, (slabs, 2 * m1, cols))
    md = torch.from_numpy(modes).cuda()
    back = torch.empty_like(xd)
    assert lib.spx_pruned_columns(3, _ptr(md), _ptr(back), n, cols, slabs, m1, 0, 1,
                                  None) == SPX_OK
    torch.cuda.synchronize()
    assert_transform_close(kept, full[:, rows, :], n, axes=(-2,))
    padded = np.zeros((slabs, n, cols), dtype=np.complex64)
    padded[:, rows, :] = modes
    assert_transform_close(back, _fft_columns(padded, True), n, axes=(-2,))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [256, 512, 1024, 2048, 4096, 8192])
def test_direct_pruned_r2c_at_every_row_width(lib, rng, n):
    # R2C rows of 16 .. 256 lanes at radix 8: the register combine with the staged store (16, 32
    # lanes) and with the direct store (64 lanes and more), each keeping 1 .. n/2 + 1 bins; a batch
    # of 37 rows leaves the last workgroup partly empty.
    from oracle import reference as ref
    from oracle.tolerance import assert_transform_close, random_real

    batch, m = 37, n // 2
    x = random_real(rng, (batch, n))
    xd = torch.from_numpy(x).cuda()
    full = ref.rfft(x)
    for keep in (1, 7, m // 2, m, m + 1):
        yd = torch.empty(batch, keep, dtype=torch.complex64, device="cuda")
        assert lib.spx_pruned_r2c(3, _ptr(xd), _ptr(yd), n, batch, keep, None) == SPX_OK
        torch.cuda.synchronize()
        assert_transform_close(yd, full[:, :keep], n)


def test_mode_gather_and_scatter_reject_bad_shapes(lib):
    # Checked on the host before any launch, so these need no GPU: each would otherwise index
    # outside the arrays.
    p = ctypes.c_void_p(0x1000)
    q = ctypes.c_void_p(0x100000)
    for fn in (lib.spx_gather_modes, lib.spx_scatter_modes):
        name = "gather_modes" if fn is lib.spx_gather_modes else "scatter_modes"
        # (n1, w, m1, m2, batch)
        for bad in [(8, 5, 2, 3, -1), (8, 5, 2, 3, 0), (0, 5, 1, 3, 1), (8, 0, 1, 1, 1),
                    (8, 5, -1, 3, 1), (8, 5, 5, 3, 1), (8, 5, 2, 0, 1), (8, 5, 2, -2, 1),
                    (8, 5, 2, 6, 1)]:
            assert fn(p, q, *bad, None) == SPX_EINVAL, bad
            assert name in _last(lib), (bad, _last(lib))


def _golden_cases():
    import json

    return json.loads((REPO / "tests" / "golden" / "modes_index.json").read_text())


@pytest.mark.gpu
@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: f"{c['n1']}x{c['n2']}-"
                         f"{c['m1']}-{c['m2']}")
def test_mode_gather_and_scatter_are_the_golden_layout(lib, case):
    # Integer-valued spectra (every value exact in float32): the gather must pick exactly the
    # fixture's positions, and the scatter must put each mode back there with zeros everywhere
    # else, bit for bit.
    n1, n2, m1, m2 = case["n1"], case["n2"], case["m1"], case["m2"]
    w = n2 // 2 + 1
    pos = np.array(case["positions"])
    batch = 3
    flat = np.arange(batch * n1 * w, dtype=np.float32)
    full = (flat + 1j * (flat % 977 - 488)).astype(np.complex64).reshape(batch, n1 * w)
    fd = torch.from_numpy(full).cuda()
    md = torch.full((batch, 2 * m1 * m2), 7 + 7j, dtype=torch.complex64, device="cuda")
    assert lib.spx_gather_modes(_ptr(fd), _ptr(md), n1, w, m1, m2, batch, None) == SPX_OK
    back = torch.full((batch, n1 * w), 5 - 5j, dtype=torch.complex64, device="cuda")
    assert lib.spx_scatter_modes(_ptr(md), _ptr(back), n1, w, m1, m2, batch, None) == SPX_OK
    torch.cuda.synchronize()
    assert torch.equal(md.cpu(), torch.from_numpy(full[:, pos]))
    expected = np.zeros_like(full)
    expected[:, pos] = full[:, pos]
    assert torch.equal(back.cpu(), torch.from_numpy(expected))


@pytest.mark.gpu
@pytest.mark.parametrize(("n1", "w", "m1", "m2"), [(1, 4096, 0, 33), (1, 7, 0, 7), (4, 3, 0, 2),
                                                   (4096, 2, 2048, 2), (6, 70, 1, 65)])
def test_mode_gather_and_scatter_edges(lib, rng, n1, w, m1, m2):
    # m1 = 0 keeps every row (the 1D pruned layout), every row kept (2 m1 = n1), rows wider than
    # a wave, and a non-power-of-two n1.
    batch = 5
    full = (rng.integers(-99, 99, (batch, n1, w)) + 1j * rng.integers(-99, 99, (batch, n1, w)))
    full = full.astype(np.complex64)
    rows = np.r_[0:m1, n1 - m1:n1] if m1 else np.arange(n1)
    expect_modes = full[:, rows, :m2]
    fd = torch.from_numpy(full).cuda()
    md = torch.empty((batch, len(rows), m2), dtype=torch.complex64, device="cuda")
    assert lib.spx_gather_modes(_ptr(fd), _ptr(md), n1, w, m1, m2, batch, None) == SPX_OK
    back = torch.full_like(fd, 3 + 3j)
    assert lib.spx_scatter_modes(_ptr(md), _ptr(back), n1, w, m1, m2, batch, None) == SPX_OK
    torch.cuda.synchronize()
    assert torch.equal(md.cpu(), torch.from_numpy(expect_modes))
    expected = np.zeros_like(full)
    expected[:, rows, :m2] = expect_modes
    assert torch.equal(back.cpu(), torch.from_numpy(expected))


@pytest.mark.gpu
@pytest.mark.parametrize(("rows", "cols", "batch"), [(1, 1, 3), (64, 64, 2), (65, 63, 3),
                                                     (1024, 16384, 1), (3, 200, 7), (513, 1, 2),
                                                     (4, 3, 4096), (31, 40, 5), (1000, 20, 2),
                                                     (32, 32, 3), (128, 65, 5), (65, 128, 5),
                                                     (257, 512, 2), (512, 257, 2), (65, 65, 3),
                                                     (129, 193, 2), (33, 65, 3), (65, 40, 3),
                                                     (193, 65, 3), (65, 193, 3), (193, 129, 2),
                                                     (79, 129, 3), (80, 128, 2), (100, 100, 3)])
def test_transpose_is_exact(lib, rng, rows, cols, batch):
    # Partial tiles on both axes, a single column or row, and a 1024 x 16384 matrix; arrays
    # with fewer than 32 rows or columns take the flat path (4 x 3: a 4 x 4 real transform's).
    # Sizes of 64k + 1 (a real spectrum's n/2 + 1) have their last row or column copied by the
    # last full tile's workgroup, alone (128 x 65, 193 x 65, 65 x 193, 257 x 512), with the other
    # axis full or partial, and both at once (65 x 65, 193 x 129, 129 x 193).
    x = (rng.standard_normal((batch, rows, cols)) + 1j * rng.standard_normal((batch, rows, cols)))
    xd = torch.from_numpy(x.astype(np.complex64)).cuda()
    yd = torch.empty(batch, cols, rows, dtype=torch.complex64, device="cuda")
    assert lib.spx_transpose(_ptr(xd), _ptr(yd), rows, cols, batch, None) == SPX_OK
    torch.cuda.synchronize()
    assert torch.equal(yd.cpu(), xd.cpu().transpose(1, 2).contiguous())


def _loaded_hip_runtime() -> ctypes.CDLL:
    # The HIP runtime this process already mapped (the one the library and PyTorch call).
    for line in Path("/proc/self/maps").read_text().splitlines():
        path = line.split()[-1]
        if "libamdhip64.so" in path:
            return ctypes.CDLL(path)
    return ctypes.CDLL("libamdhip64.so")


@pytest.mark.gpu
def test_large_transforms_keep_their_workspace_in_the_retained_pool(lib, rng):
    # A 2^20-point transform takes its scratch from the default pool in stream order; the first
    # such call raises the pool's release threshold, so after a synchronization the freed scratch
    # stays reserved for the next call instead of going back to the driver.
    from oracle import reference as ref
    from oracle.tolerance import assert_transform_close, random_complex

    n = 1 << 20
    x = random_complex(rng, (2, n))
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    assert lib.spx_c2c(3, _ptr(xd), _ptr(yd), n, 2, 0, None) == SPX_OK, _last(lib)
    torch.cuda.synchronize()
    hip = _loaded_hip_runtime()
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), torch.cuda.current_device()) == 0
    threshold = ctypes.c_uint64()
    assert hip.hipMemPoolGetAttribute(pool, 4, ctypes.byref(threshold)) == 0  # ReleaseThreshold
    assert threshold.value == 2**64 - 1
    reserved = ctypes.c_uint64()
    assert hip.hipMemPoolGetAttribute(pool, 5, ctypes.byref(reserved)) == 0  # ReservedMemCurrent
    assert reserved.value >= 2 * n * 8
    assert_transform_close(yd, ref.fft(x), n)


def test_noalloc_c2c_rejects_what_its_static_scratch_cannot_hold(lib):
    # Checked on the host before anything is queued: more than 2^22 values of scratch, and the
    # table variant (whose first call allocates its table).
    p = ctypes.c_void_p(0x1000)
    q = ctypes.c_void_p(0x10000000)
    assert lib.spx_c2c_noalloc(3, p, q, 1 << 20, 5, 0, None) == SPX_EINVAL
    assert "split the batch" in _last(lib)
    assert lib.spx_c2c_noalloc(3, p, q, 1 << 24, 1, 0, None) == SPX_EINVAL
    info = Info()
    lazy = []
    for impl in range(lib.spx_impl_count()):
        assert lib.spx_impl_get_info(impl, ctypes.byref(info)) == SPX_OK
        if info.lazy_table:
            lazy.append(impl)
    assert lazy, "the registry has a table variant"
    for impl in lazy:  # refused at every size, before the table could be built
        for n, batch in [(1 << 20, 1), (1024, 8), (2, 1)]:
            assert lib.spx_c2c_noalloc(impl, p, q, n, batch, 0, None) == SPX_EINVAL
            assert "twiddle table" in _last(lib)
    assert lib.spx_c2c_noalloc(3, p, q, 3 << 20, 1, 0, None) == SPX_EINVAL
    assert "power of two" in _last(lib)
    assert lib.spx_c2c_noalloc(3, p, q, 1 << 20, 0, 0, None) == SPX_EINVAL
