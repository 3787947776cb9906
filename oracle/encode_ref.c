/*
 * Plain-C float64 brute-force block-VQ encoder.  TEST INFRASTRUCTURE ONLY:
 * a CPU restatement used to check the HIP encoder, never shipped.
 *
 * Restates SunShapeBlockCodec.quantize (reference codec.py:424-470) and the
 * encode kernel body (reference kernels.py:1013-1024): for every token and
 * block, the centroid minimising sum_d (k_d - c_d)^2, with a strict '<' so
 * that ties keep the lowest index (kernels.py:1020).  Arithmetic is float64
 * (the reference's float32 fast-math rounding is not pinned); a (token, block)
 * is flagged as a near-tie when a centroid with a different vector lies within
 * near_rel (relative) of the best distance.
 *
 * Same contract as oracle/sunshape_oracle.py:encode_blockvq; the two are
 * cross-checked in tests/test_oracle_encode.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* keys: n x d float32, already permuted; cents: nb x nc x bd float32. */
int ss_oracle_encode(const float *keys, long n, int d, const float *cents,
                     int nb, int nc, int bd, double near_rel,
                     int32_t *out_idx, uint8_t *out_near)
{
    if (nb * bd != d || nc <= 0 || nc > 65536)
        return -1;
    int *dup = (int *)malloc(sizeof(int) * (size_t)nb * nc);
    if (!dup)
        return -2;
    /* dup[b][c] = lowest centroid index with a bit-identical vector */
    for (int b = 0; b < nb; ++b) {
        const float *cb = cents + (size_t)b * nc * bd;
        for (int c = 0; c < nc; ++c) {
            int id = c;
            for (int c2 = 0; c2 < c; ++c2) {
                if (memcmp(cb + (size_t)c2 * bd, cb + (size_t)c * bd,
                           sizeof(float) * bd) == 0) {
                    id = c2;
                    break;
                }
            }
            dup[b * nc + c] = id;
        }
    }
#pragma omp parallel for schedule(static)
    for (long t = 0; t < n; ++t) {
        double dist[4096];
        double *dd = dist;
        double *heap = NULL;
        if (nc > 4096) {
            heap = (double *)malloc(sizeof(double) * nc);
            dd = heap;
        }
        for (int b = 0; b < nb; ++b) {
            const float *kb = keys + (size_t)t * d + (size_t)b * bd;
            const float *cb = cents + (size_t)b * nc * bd;
            double best = 0.0;
            int best_i = 0;
            for (int c = 0; c < nc; ++c) {
                double acc = 0.0;
                for (int j = 0; j < bd; ++j) {
                    double df = (double)kb[j] - (double)cb[(size_t)c * bd + j];
                    acc += df * df;
                }
                dd[c] = acc;
                if (c == 0 || acc < best) {
                    best = acc;
                    best_i = c;
                }
            }
            uint8_t near = 0;
            const double lim = best * (1.0 + near_rel);
            for (int c = 0; c < nc; ++c) {
                if (dup[b * nc + c] != dup[b * nc + best_i] && dd[c] <= lim) {
                    near = 1;
                    break;
                }
            }
            out_idx[(size_t)t * nb + b] = best_i;
            out_near[(size_t)t * nb + b] = near;
        }
        free(heap);
    }
    free(dup);
    return 0;
}
