// Pruned transforms for the FNO mode layout (the contract of reference pruned.hpp:3-17):
//
//   1D complex  forward keeps the first `keep` outputs; inverse reads `keep` inputs, the rest zero.
//   2D real     of rfft2's n1 x (n2/2 + 1) half spectrum, rows 0 .. m1-1 then n1-m1 .. n1-1 and
//               columns 0 .. m2-1, as a (2 m1) x m2 block; the inverse zero-fills the rest.
//
// A 2D request is planned once (ModesPlan): its route and workspace.
//
//   SinglePass   one kernel per array, the tile in LDS (fft2_fused.hpp / fft2_modes.hpp)
//   InKernel     pruned real rows that write only m2 columns, then pruned columns that keep
//                only the 2 m1 rows (the inverse mirrored), through an n1 x m2 workspace
//   Transposes   implementations without pruned kernels (naive): the mode selection is folded
//                into the transposes of the transpose method. Forward: real rows (n1 x w), a
//                transpose that keeps only the m2 kept columns (m2 x n1), the column transforms
//                of those alone, and a transpose that gathers the kept rows straight into the
//                mode block. Inverse: a transpose that scatters the mode block into m2 x n1
//                column inputs (zeros in the dropped rows, written in the same pass), their
//                inverse transforms, a transpose back that zero-extends to n1 x w, the real rows.
//                No full-spectrum gather or scatter pass, and w / m2 times fewer column
//                transforms than a full transform.
//
// gather_modes / scatter_modes (the C ABI's) are single row remaps between a full half spectrum
// and a mode block; the scatter writes every value of the full spectrum once.

#include "fft_api.hpp"

#include <algorithm>
#include <climits>

namespace spx {
namespace {

std::size_t values(long long rows, long long cols, long long batch)
{
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(rows)
           * static_cast<std::size_t>(cols);
}

// Throws `InvalidArgument(what())` unless ok.
template <class Message>
void expect(bool ok, Message&& what)
{
    if (!ok) {
        throw InvalidArgument(what());
    }
}

enum class ModesRoute { SinglePass, InKernel, Transposes };

struct ModesPlan {
    ModesRoute route;
    int n1;
    int n2;
    int m1;
    int m2;
    int batch;
    int w;               // n2 / 2 + 1
    std::size_t full;    // n1 x w per array: the real rows' output (Transposes)
    std::size_t narrow;  // n1 x m2 per array: the kept columns
    std::size_t real;    // scratch of the generic real rows

    std::size_t words() const
    {
        switch (route) {
        case ModesRoute::SinglePass: return 0;
        case ModesRoute::InKernel: return narrow;
        default: return full + narrow + real;
        }
    }
};

// The argument rules and their messages are the reference's API (pruned.cu:78-111).
ModesPlan plan_modes(const FftImpl& impl, int n1, int n2, int m1, int m2, int batch)
{
    const std::string name = impl.name;
    expect(is_pow2(n1) && n1 <= impl.max_n, [&] {
        return "rfft2 modes: " + name + " needs n1 to be a power of two up to " + str(impl.max_n)
               + ", got " + str(n1);
    });
    expect(is_pow2(n2) && n2 >= 2 && n2 <= impl.max_real_n, [&] {
        return "rfft2 modes: " + name + " needs n2 to be a power of two from 2 up to "
               + str(impl.max_real_n) + ", got " + str(n2);
    });
    expect(m1 >= 1 && 2 * m1 <= n1 && m2 >= 1 && m2 <= n2 / 2 + 1, [&] {
        return "rfft2 modes: need 1 <= m1 <= n1/2 and 1 <= m2 <= n2/2 + 1, got m1 = " + str(m1)
               + ", m2 = " + str(m2) + " for " + str(n1) + " x " + str(n2);
    });
    expect(batch >= 1 && static_cast<long long>(batch) * std::max(n1, n2) <= INT_MAX,
           [] { return std::string("rfft2 modes: batch out of range"); });

    ModesPlan p{ModesRoute::Transposes, n1, n2, m1, m2, batch, n2 / 2 + 1, 0, 0, 0};
    p.narrow = values(n1, m2, batch);
    if (impl.fused != nullptr && impl.fused->supports(n1, n2)) {
        p.route = ModesRoute::SinglePass;
    } else if (impl.pruned != nullptr) {
        p.route = ModesRoute::InKernel;
    } else {
        p.full = values(n1, p.w, batch);
        p.real = impl.real_needs_work ? values(n1, n2 / 2, batch) : 0;
    }
    return p;
}

void check_1d(const FftImpl& impl, int n, int keep, int batch)
{
    expect(is_pow2(n) && n <= impl.max_n, [&] {
        return "fft_c2c_pruned: " + std::string(impl.name) + " needs n to be a power of two up to "
               + str(impl.max_n) + ", got " + str(n);
    });
    expect(keep >= 1 && keep <= n, [&] {
        return "fft_c2c_pruned: keep must be in [1, " + str(n) + "], got " + str(keep);
    });
    expect(batch >= 1, [] { return std::string("fft_c2c_pruned: batch must be at least 1"); });
}

// The mode block's shape against the full spectrum's: m1 = 0 keeps all n1 rows.
void check_band(int n1, int w, int m1, int m2, int batch, const char* who)
{
    expect(n1 >= 1 && w >= 1 && batch >= 1, [&] {
        return std::string(who) + ": need n1, w and batch >= 1, got n1 = " + str(n1) + ", w = "
               + str(w) + ", batch = " + str(batch);
    });
    expect(m1 >= 0 && 2LL * m1 <= n1 && m2 >= 1 && m2 <= w, [&] {
        return std::string(who) + ": need 0 <= m1 <= n1/2 and 1 <= m2 <= w, got m1 = " + str(m1)
               + ", m2 = " + str(m2) + " for " + str(n1) + " x " + str(w);
    });
}

int kept_rows(int n1, int m1) { return m1 > 0 ? 2 * m1 : n1; }

void gather(const cf32* full, cf32* modes, int n1, int w, int m1, int m2, int batch,
            hipStream_t stream)
{
    const Remap r{kept_rows(n1, m1), m2, w, static_cast<long long>(n1) * w, batch,
                  AxisMap::keep(n1, m1), AxisMap::identity(m2)};
    remap(full, modes, r, false, stream);
}

void scatter(const cf32* modes, cf32* full, int n1, int w, int m1, int m2, int batch,
             hipStream_t stream)
{
    const Remap r{n1, w, m2, static_cast<long long>(kept_rows(n1, m1)) * m2, batch,
                  AxisMap::spread(n1, m1), AxisMap::identity(m2)};
    remap(modes, full, r, false, stream);
}

}  // namespace

void gather_modes(const cf32* full, cf32* modes, int n1, int w, int m1, int m2, int batch,
                  hipStream_t stream)
{
    check_band(n1, w, m1, m2, batch, "gather_modes");
    gather(full, modes, n1, w, m1, m2, batch, stream);
}

void scatter_modes(const cf32* modes, cf32* full, int n1, int w, int m1, int m2, int batch,
                   hipStream_t stream)
{
    check_band(n1, w, m1, m2, batch, "scatter_modes");
    scatter(modes, full, n1, w, m1, m2, batch, stream);
}

std::size_t fft_c2c_pruned_workspace(const FftImpl& impl, int n, int, int batch)
{
    return impl.pruned != nullptr ? 0 : values(1, n, batch);
}

void fft_c2c_pruned(const FftImpl& impl, const cf32* x, cf32* y, int n, int keep, int batch,
                    Direction direction, cf32* work, hipStream_t stream)
{
    check_1d(impl, n, keep, batch);
    if (impl.pruned != nullptr) {
        impl.pruned->c2c(x, y, n, batch, keep, direction, stream);
        return;
    }
    // A row of n values per transform, of which the first keep are the modes.
    if (direction == Direction::Forward) {
        impl.c2c(x, work, n, batch, direction, stream);
        gather(work, y, 1, n, 0, keep, batch, stream);
    } else {
        scatter(x, work, 1, n, 0, keep, batch, stream);
        impl.c2c(work, y, n, batch, direction, stream);
    }
}

std::size_t rfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int m1, int m2, int batch)
{
    return plan_modes(impl, n1, n2, m1, m2, batch).words();
}

std::size_t irfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int m1, int m2,
                                   int batch)
{
    return plan_modes(impl, n1, n2, m1, m2, batch).words();
}

void rfft2_modes(const FftImpl& impl, const float* x, cf32* modes, int n1, int n2, int m1,
                 int m2, int batch, cf32* work, hipStream_t stream)
{
    const ModesPlan p = plan_modes(impl, n1, n2, m1, m2, batch);
    if (p.route == ModesRoute::SinglePass) {
        impl.fused->r2c(x, modes, n1, n2, m1, m2, batch, stream);
        return;
    }
    if (p.route == ModesRoute::InKernel) {
        impl.pruned->r2c_work(x, work, n2, batch * n1, m2, stream);  // n1 x m2 per array
        impl.pruned->columns(work, modes, n1, m2, batch, 0, m1, Direction::Forward, stream);
        return;
    }
    cf32* rows = work;              // n1 x w, later the column transforms' output (m2 x n1)
    cf32* cols = work + p.full;     // m2 x n1: the kept columns, transposed
    cf32* scratch = p.real > 0 ? cols + p.narrow : nullptr;
    impl.r2c(x, rows, n2, batch * n1, scratch, stream);
    // cols[c][i] = rows[i][c] for the kept c < m2 only
    remap(rows, cols,
          Remap{m2, n1, p.w, static_cast<long long>(n1) * p.w, batch, AxisMap::identity(n1),
                AxisMap::identity(m2)},
          true, stream);
    impl.c2c(cols, rows, n1, batch * m2, Direction::Forward, stream);
    // modes[r][c] = rows[c][keep(r)]: the transpose back gathers the kept frequencies
    remap(rows, modes,
          Remap{2 * m1, m2, n1, static_cast<long long>(m2) * n1, batch, AxisMap::identity(m2),
                AxisMap::keep(n1, m1)},
          true, stream);
}

void irfft2_modes(const FftImpl& impl, const cf32* modes, float* y, int n1, int n2, int m1,
                  int m2, int batch, cf32* work, hipStream_t stream)
{
    const ModesPlan p = plan_modes(impl, n1, n2, m1, m2, batch);
    if (p.route == ModesRoute::SinglePass) {
        impl.fused->c2r(modes, y, n1, n2, m1, m2, batch, stream);
        return;
    }
    if (p.route == ModesRoute::InKernel) {
        impl.pruned->columns_work(modes, work, n1, m2, batch, m1, 0, Direction::Inverse, stream);
        impl.pruned->c2r(work, y, n2, batch * n1, m2, stream);  // columns m2.. are zero
        return;
    }
    cf32* rows = work;           // first the scattered column inputs (m2 x n1), then n1 x w
    cf32* cols = work + p.full;  // the column transforms' output (m2 x n1)
    cf32* scratch = p.real > 0 ? cols + p.narrow : nullptr;
    // rows[c][i] = modes[spread(i)][c], zero for a dropped frequency row i
    remap(modes, rows,
          Remap{m2, n1, m2, static_cast<long long>(2 * m1) * m2, batch,
                AxisMap::spread(n1, m1), AxisMap::identity(m2)},
          true, stream);
    impl.c2c(rows, cols, n1, batch * m2, Direction::Inverse, stream);
    // rows[i][c] = cols[c][i] for c < m2, zero for the dropped columns m2 .. w-1
    remap(cols, rows,
          Remap{n1, p.w, n1, static_cast<long long>(m2) * n1, batch, AxisMap::identity(m2),
                AxisMap::identity(n1)},
          true, stream);
    impl.c2r(rows, y, n2, batch * n1, scratch, stream);
}

}  // namespace spx
