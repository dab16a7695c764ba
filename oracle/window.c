/*
 * Oracle: plain-C restatement of the reference's neighbourhood window rule
 * and flattened index maps.  TEST INFRASTRUCTURE ONLY -- loaded by tests/
 * through ctypes, never linked into the shipped library.
 *
 *   oracle_window_start   utils/window.py:91-111 (scalar rule; same values as
 *                         the vectorised form at utils/window.py:6-46)
 *   oracle_axis_map       _core/pure.py:27-56   (non-causal / causal axis map)
 *   oracle_neighborhood   _core/pure.py:91-129, 335-387 (flattened map over
 *                         up to three axes, row-major kernel order)
 *
 * Paths are relative to /root/reference/src/natten_mps.
 */
#include <stdint.h>
#include <stdlib.h>

int64_t oracle_window_start(int64_t i, int64_t L, int64_t K, int64_t d)
{
    const int64_t half = K / 2;
    if (d <= 1) {
        int64_t s = i - half;
        if (s < 0) s = 0;
        if (i + half >= L) s += L - i - half - 1;
        return s;
    }
    if (i - half * d < 0) return i % d;
    if (i + half * d >= L) {
        const int64_t r = i % d;
        const int64_t full = (L / d) * d;
        const int64_t tail = L - full;
        if (r < tail) return L - tail + r - 2 * half * d;
        return full + r - K * d;
    }
    return i - half * d;
}

/* One axis: query positions pos[o] = o*s for o < n_out.  idx/valid are
 * [n_out][K].  Causal indices are clamped to [0, L-1] exactly as the
 * reference clamps them; validity is 0 <= raw <= pos. */
void oracle_axis_map(int64_t L, int64_t K, int64_t d, int64_t s, int causal,
                     int64_t n_out, int64_t *idx, uint8_t *valid)
{
    for (int64_t o = 0; o < n_out; ++o) {
        const int64_t p = o * s;
        const int64_t first = causal ? p - (K - 1) * d : oracle_window_start(p, L, K, d);
        for (int64_t k = 0; k < K; ++k) {
            int64_t raw = first + k * d;
            uint8_t ok = 1;
            if (causal) {
                ok = (raw >= 0) && (raw <= p);
                if (raw < 0) raw = 0;
                if (raw > L - 1) raw = L - 1;
            }
            idx[o * K + k] = raw;
            valid[o * K + k] = ok;
        }
    }
}

/* Three axes (outermost first).  Unused axes are passed as len=1, K=1,
 * d=1, s=1, causal=0.  flat/valid are [n0][n1][n2][K0*K1*K2]. */
void oracle_neighborhood(const int64_t len[3], const int64_t K[3], const int64_t d[3],
                         const int64_t s[3], const int causal[3],
                         int64_t *flat, uint8_t *valid)
{
    int64_t n[3];
    for (int a = 0; a < 3; ++a) n[a] = (len[a] + s[a] - 1) / s[a];
    const int64_t kv = K[0] * K[1] * K[2];
    int64_t *i0 = malloc(sizeof(int64_t) * (size_t)(n[0] * K[0]));
    int64_t *i1 = malloc(sizeof(int64_t) * (size_t)(n[1] * K[1]));
    int64_t *i2 = malloc(sizeof(int64_t) * (size_t)(n[2] * K[2]));
    uint8_t *v0 = malloc((size_t)(n[0] * K[0]));
    uint8_t *v1 = malloc((size_t)(n[1] * K[1]));
    uint8_t *v2 = malloc((size_t)(n[2] * K[2]));
    oracle_axis_map(len[0], K[0], d[0], s[0], causal[0], n[0], i0, v0);
    oracle_axis_map(len[1], K[1], d[1], s[1], causal[1], n[1], i1, v1);
    oracle_axis_map(len[2], K[2], d[2], s[2], causal[2], n[2], i2, v2);
    int64_t q = 0;
    for (int64_t a = 0; a < n[0]; ++a)
        for (int64_t b = 0; b < n[1]; ++b)
            for (int64_t c = 0; c < n[2]; ++c, ++q) {
                int64_t e = 0;
                for (int64_t x = 0; x < K[0]; ++x)
                    for (int64_t y = 0; y < K[1]; ++y)
                        for (int64_t z = 0; z < K[2]; ++z, ++e) {
                            const int64_t f = (i0[a * K[0] + x] * len[1] + i1[b * K[1] + y]) * len[2]
                                              + i2[c * K[2] + z];
                            flat[q * kv + e] = f;
                            valid[q * kv + e] = v0[a * K[0] + x] & v1[b * K[1] + y] & v2[c * K[2] + z];
                        }
            }
    free(i0); free(i1); free(i2); free(v0); free(v1); free(v2);
}
