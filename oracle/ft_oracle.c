/*
 * CPU oracle for the sparse feature-transformer (FT) path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C on the CPU, the
 * arithmetic of the reference FT op so that the HIP kernels can be checked
 * against it.  It is never linked into, called by, or used as a fallback for
 * the product library: only tests, the smoke check and the CPU-baseline leg
 * of the benchmark may load it.
 *
 * Reference paths are relative to the root of rgodha24/stockfish-trainer;
 * FT/ = src/model/modules/feature_transformer/.
 *
 * Index contract (all functions): idx is int32 [B, K] row-major; a slot equal
 * to -1 is inactive wherever it sits in the row (FT/kernel.py:97-98).  Any
 * other value outside [0, N) is undefined behaviour in the reference; here it
 * makes the function return ORACLE_EBADIDX without writing the outputs.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).  Results do not
 * depend on the thread count: every float sequence that is summed is summed by
 * one thread in the fixed order stated at each function.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EBADIDX (-1)
#define ORACLE_ENOMEM (-2)
#define ORACLE_EARG (-3)

static int check_indices(const int32_t *idx, int64_t n, int64_t num_inputs) {
    for (int64_t i = 0; i < n; ++i) {
        int32_t v = idx[i];
        if (v != -1 && (v < 0 || (int64_t)v >= num_inputs)) return ORACLE_EBADIDX;
    }
    return ORACLE_OK;
}

int oracle_abi_version(void) { return 1; }

/*
 * fp32 forward in the reference's order (FT/kernel.py:89-103, K1):
 *   acc = bias[c]; for k = 0..K-1: if idx[b,k] != -1: acc += W[idx[b,k], c]
 *   out[b, c] = acc
 * Every add is one IEEE-754 binary32 add, in that order (no FMA, no reassoc).
 */
int oracle_ft_fwd_f32(const int32_t *idx, int64_t B, int32_t K, const float *W, int64_t N,
                      int32_t L, const float *bias, float *out) {
    if (B < 0 || K <= 0 || N <= 0 || L <= 0) return ORACLE_EARG;
    if (check_indices(idx, B * (int64_t)K, N) != ORACLE_OK) return ORACLE_EBADIDX;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        float *o = out + b * (int64_t)L;
        for (int32_t c = 0; c < L; ++c) o[c] = bias[c];
        const int32_t *row = idx + b * (int64_t)K;
        for (int32_t k = 0; k < K; ++k) {
            int32_t f = row[k];
            if (f == -1) continue;
            const float *w = W + (int64_t)f * L;
            for (int32_t c = 0; c < L; ++c) o[c] = o[c] + w[c];
        }
    }
    return ORACLE_OK;
}

/* Same sum in binary64 (inputs widened exactly); the tolerance reference. */
int oracle_ft_fwd_f64(const int32_t *idx, int64_t B, int32_t K, const float *W, int64_t N,
                      int32_t L, const float *bias, double *out) {
    if (B < 0 || K <= 0 || N <= 0 || L <= 0) return ORACLE_EARG;
    if (check_indices(idx, B * (int64_t)K, N) != ORACLE_OK) return ORACLE_EBADIDX;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        double *o = out + b * (int64_t)L;
        for (int32_t c = 0; c < L; ++c) o[c] = (double)bias[c];
        const int32_t *row = idx + b * (int64_t)K;
        for (int32_t k = 0; k < K; ++k) {
            int32_t f = row[k];
            if (f == -1) continue;
            const float *w = W + (int64_t)f * L;
            for (int32_t c = 0; c < L; ++c) o[c] += (double)w[c];
        }
    }
    return ORACLE_OK;
}

/*
 * fp32 backward in the reference's order.
 *   Weight grad (FT/kernel.py:108-138 then K2 FT/kernel.py:167-186): the flat
 *   (b, k) slots are stably sorted by feature, so for each feature f present in
 *   idx the grad rows are summed in ascending flat order b*K+k onto acc = 0.0f,
 *   then dW[f, c] = dW[f, c] + acc[c].  Rows of features that never occur are
 *   not touched.  Walking the slots once in flat order and adding G[b] into
 *   acc[f] reproduces each feature's sequence exactly.
 *   Bias grad (FT/kernel.py:269): db[c] = db[c] + sum_b G[b, c].  torch's
 *   reduction order is not part of the contract, so the column sum is formed
 *   in binary64 and rounded once to binary32 before the add.
 * Threads split the columns; each column's sequence stays in one thread.
 */
int oracle_ft_bwd_f32(const int32_t *idx, int64_t B, int32_t K, const float *G, int64_t N,
                      int32_t L, float *dW, float *db) {
    if (B < 0 || K <= 0 || N <= 0 || L <= 0) return ORACLE_EARG;
    if (check_indices(idx, B * (int64_t)K, N) != ORACLE_OK) return ORACLE_EBADIDX;
    float *acc = (float *)calloc((size_t)N * (size_t)L, sizeof(float));
    unsigned char *present = (unsigned char *)calloc((size_t)N, 1);
    if (!acc || !present) {
        free(acc);
        free(present);
        return ORACLE_ENOMEM;
    }
    for (int64_t s = 0; s < B * (int64_t)K; ++s)
        if (idx[s] != -1) present[idx[s]] = 1;

    const int32_t CB = 64; /* column block per task */
    int32_t nblk = (L + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int32_t blk = 0; blk < nblk; ++blk) {
        int32_t c0 = blk * CB, c1 = c0 + CB < L ? c0 + CB : L;
        for (int64_t b = 0; b < B; ++b) {
            const float *g = G + b * (int64_t)L;
            const int32_t *row = idx + b * (int64_t)K;
            for (int32_t k = 0; k < K; ++k) {
                int32_t f = row[k];
                if (f == -1) continue;
                float *a = acc + (int64_t)f * L;
                for (int32_t c = c0; c < c1; ++c) a[c] = a[c] + g[c];
            }
        }
        for (int64_t f = 0; f < N; ++f) {
            if (!present[f]) continue;
            float *d = dW + f * (int64_t)L;
            const float *a = acc + f * (int64_t)L;
            for (int32_t c = c0; c < c1; ++c) d[c] = d[c] + a[c];
        }
        for (int32_t c = c0; c < c1; ++c) {
            double s = 0.0;
            for (int64_t b = 0; b < B; ++b) s += (double)G[b * (int64_t)L + c];
            db[c] = db[c] + (float)s;
        }
    }
    free(acc);
    free(present);
    return ORACLE_OK;
}

/* Backward in binary64: dW[f] += sum of G rows over slots with feature f; db += colsum. */
int oracle_ft_bwd_f64(const int32_t *idx, int64_t B, int32_t K, const float *G, int64_t N,
                      int32_t L, double *dW, double *db) {
    if (B < 0 || K <= 0 || N <= 0 || L <= 0) return ORACLE_EARG;
    if (check_indices(idx, B * (int64_t)K, N) != ORACLE_OK) return ORACLE_EBADIDX;
    const int32_t CB = 64;
    int32_t nblk = (L + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int32_t blk = 0; blk < nblk; ++blk) {
        int32_t c0 = blk * CB, c1 = c0 + CB < L ? c0 + CB : L;
        for (int64_t b = 0; b < B; ++b) {
            const float *g = G + b * (int64_t)L;
            const int32_t *row = idx + b * (int64_t)K;
            for (int32_t k = 0; k < K; ++k) {
                int32_t f = row[k];
                if (f == -1) continue;
                double *d = dW + (int64_t)f * L;
                for (int32_t c = c0; c < c1; ++c) d[c] += (double)g[c];
            }
        }
        for (int32_t c = c0; c < c1; ++c) {
            double s = 0.0;
            for (int64_t b = 0; b < B; ++b) s += (double)G[b * (int64_t)L + c];
            db[c] += s;
        }
    }
    return ORACLE_OK;
}

/*
 * Quantized (int16-weight) FT forward.  The reference has no quantized forward
 * (the Stockfish engine that holds one is an empty submodule); this restates
 * the integer closed form the export feeds (src/model/quantize.py:76-93,
 * src/scripts/serialize.py:199-226):
 *   acc[b, c] = bq[c] + sum_{k active} Wq[idx[b,k], c]        (exact int32)
 *   if wrap16: acc = (int16_t)acc  (two's-complement wrap, i.e. an int16
 *              accumulator with wrapping adds, since reduction mod 2^16 is a
 *              ring homomorphism)
 *   out[b, c] = clamp(acc, clip_lo, clip_hi) as int16
 *   psqt_out[b, p] = sum_{k active} psqt[idx[b,k], p]  (int32, no bias)
 * psqt / psqt_out may be NULL (P ignored).  The int32 sum cannot overflow for
 * K < 65536 because every term lies in [-32768, 32767].
 */
int oracle_ft_fwd_i16(const int32_t *idx, int64_t B, int32_t K, const int16_t *Wq, int64_t N,
                      int32_t L, const int16_t *bq, const int32_t *psqt, int32_t P,
                      int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                      int32_t wrap16) {
    if (B < 0 || K <= 0 || N <= 0 || L <= 0 || K >= 65536 || clip_lo > clip_hi)
        return ORACLE_EARG;
    if (check_indices(idx, B * (int64_t)K, N) != ORACLE_OK) return ORACLE_EBADIDX;
#pragma omp parallel
    {
        int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)L);
#pragma omp for schedule(static)
        for (int64_t b = 0; b < B; ++b) {
            const int32_t *row = idx + b * (int64_t)K;
            for (int32_t c = 0; c < L; ++c) acc[c] = bq[c];
            for (int32_t k = 0; k < K; ++k) {
                int32_t f = row[k];
                if (f == -1) continue;
                const int16_t *w = Wq + (int64_t)f * L;
                for (int32_t c = 0; c < L; ++c) acc[c] += w[c];
            }
            int16_t *o = out + b * (int64_t)L;
            for (int32_t c = 0; c < L; ++c) {
                int32_t v = acc[c];
                if (wrap16) v = (int32_t)(int16_t)(uint16_t)(uint32_t)v;
                if (v < clip_lo) v = clip_lo;
                if (v > clip_hi) v = clip_hi;
                o[c] = (int16_t)v;
            }
            if (psqt && psqt_out) {
                int32_t *po = psqt_out + b * (int64_t)P;
                for (int32_t p = 0; p < P; ++p) po[p] = 0;
                for (int32_t k = 0; k < K; ++k) {
                    int32_t f = row[k];
                    if (f == -1) continue;
                    const int32_t *pw = psqt + (int64_t)f * P;
                    for (int32_t p = 0; p < P; ++p) po[p] += pw[p];
                }
            }
        }
        free(acc);
    }
    return ORACLE_OK;
}

/*
 * Weight quantization of the export path (src/model/quantize.py:83-84):
 *   q = round_half_even(float32(x * scale)), saturated to int16 when clamp != 0.
 * torch's fp32 mul then round() is binary32 multiply + round-half-to-even;
 * rintf in the default rounding mode is the same.  With clamp == 0 a value
 * outside int16 makes the function return ORACLE_EARG (the reference's
 * .to(torch.int16) of such a value is undefined).
 */
int oracle_quantize_i16(const float *x, int64_t n, float scale, int32_t clamp, int16_t *out) {
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i] * scale;
        float r = rintf(v);
        if (r < -32768.0f || r > 32767.0f) {
            if (!clamp) return ORACLE_EARG;
            r = r < 0 ? -32768.0f : 32767.0f;
        }
        out[i] = (int16_t)r;
    }
    return ORACLE_OK;
}
