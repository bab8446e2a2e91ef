"""CPU oracle for the batched-FFT hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or the timed CPU baseline), never as the thing measured or shipped: the
product path (gpu-spectral-stack_amd/) never imports it and has no CPU fallback.

Modules:
  reference  float64 NumPy transforms: the reference's oracle (python/spectral/reference.py)
  tolerance  the reference's tolerance policy and comparison helpers (python/spectral/testing.py)
  model      a NumPy model of this repository's kernels' schedule: the Stockham stage index maps
             for a (N, radix, values-per-lane) plan, the conjugate-pair real combine / prepare,
             the strided-column row map and the FNO mode index map. It pins the index logic the
             HIP kernels implement against the mathematics, on the CPU.

Pinning (what makes each function trustworthy, besides the reference's own tests):
  reference.fft/ifft/rfft/irfft/fft2/...  numpy.fft (pocketfft), itself pinned against the O(N^2)
      definition `dft` at small sizes and closed forms (impulse, tone, constant).
  reference.ifft2  the inverse definition on both axes (conjugate of `dft` applied twice),
      row-then-column ifft, fft2 round trip, and a separable tone's closed form.
  reference.fft_truncate  the first k outputs of `dft`; a tone at k - 1 peaks in the last slot.
  reference.ifft_from_modes  the inverse definition summed over the kept input frequencies one
      at a time, a unit mode's closed form e^{2 pi i k m / n} / n, and ifft_from_modes(fft(x)) = x.
      Planted mistakes (modes at the end, forward sign, unscaled) fail these checks.
  reference.rfft2_truncate / irfft2_from_modes  the frequency semantics of the FNO layout,
      pinned by a brute-force enumeration of kept frequencies and the committed fixture
      tests/golden/modes_index.json, and by the reference's own known-answer test
      (test_reference.py:53-59), restated.
  model.*  against numpy.fft and `dft` (values), and against brute-force index enumeration.
There are no golden vectors for this path in the reference (its only fixtures are RF signals,
outside this path), so no function here is pinned by reference-held vectors.
"""
