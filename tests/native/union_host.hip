// Host build of the variable-length tile sizing (union_extent_upto in
// na_tile.h) against brute force over axis_geometry (na_common.h), exported
// for the CPU tests through ctypes.
#include "na_tile.h"

extern "C" {

// For a padded extent Lmax: the largest union of any tile of T items (query
// or key side) over every sample extent from K * dil to Lmax, by brute force,
// against union_extent_upto.  Returns 1 when union_extent_upto is smaller
// (an undersized LDS slice), else 0.
int host_union_upto_undersized(int Lmax, int K, int d, int causal, int T, int key) {
    int want = 1;
    for (int L = K * d; L <= Lmax; ++L) {
        if (!causal && d == 1 && K % 2 == 0 && K == L) continue;
        const na::FastDiv fd = na::make_fastdiv(static_cast<uint32_t>(d));
        for (int r = 0; r < d && r < L; ++r) {
            const int cn = (L - r + d - 1) / d;
            for (int t = 0; t * T < cn; ++t) {
                const na::AxisGeo g = na::axis_geometry(L, K, d, causal, L % d, 1, L, T, t, r, 0, T - 1, key != 0, fd);
                if (g.U > want) want = g.U;
            }
        }
    }
    const na::Axis A{Lmax, Lmax, K, d, 1, causal};
    return na::union_extent_upto(A, T, key != 0) < want ? 1 : 0;
}

}  // extern "C"
