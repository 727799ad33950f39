/* Plain-C oracle for the fused dequantize+GEMM path. TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Scalar code with wide accumulators (int64 for the integer path, double for
 * the float paths), parallelised over output rows with OpenMP. It restates:
 *   - the per-token int8 quantizer      src/lowbit/csrc/dispatch.c:231-257
 *   - exact W4A8 group accumulators     src/lowbit/reference.py:18-26,
 *                                       src/lowbit/csrc/kern_scalar.c:49-59
 *   - float64 W4A16 / MXFP4 / W4A8 GEMMs src/lowbit/reference.py:9-34
 *   - the error-bound magnitudes        tests/conftest.py:22-27,
 *                                       tests/test_kernels.py:108-116
 * Packed layouts: src/lowbit/csrc/lowbit.h:9-19.
 *
 * Build: oracle/Makefile (gcc -O2, no fast-math: the quantizer must round
 * exactly like IEEE float32).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 128
#define MXBLOCK 32

/* code of element k in a packed row with "j / j+half" blocks */
static inline int code_at(const uint8_t *row, int k, int block) {
    const int half = block / 2, b = k / block, p = k % block;
    const uint8_t byte = row[b * half + (p % half)];
    return p < half ? (byte & 15) : (byte >> 4);
}

static inline float e8m0_f32(uint8_t e) {
    if (e == 255) return NAN;
    return ldexpf(1.0f, (int)e - 127); /* e = 0 -> 2^-127, a float32 subnormal */
}

static const float E2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,
                               4.0f,  6.0f,  -0.0f, -0.5f, -1.0f, -1.5f,
                               -2.0f, -3.0f, -4.0f, -6.0f};

int orc_version(void) { return 1; }

/* xq[m,k] = clip(rint(x/sc), +-127), sc = amax/127 (1 if amax == 0); asum = group sums. */
void orc_quant_act_int8(const float *x, int M, int Kp, int8_t *xq, float *xs,
                        int32_t *asum) {
    const int G = Kp / GROUP;
    for (int m = 0; m < M; m++) {
        const float *r = x + (size_t)m * Kp;
        float amax = 0.0f;
        for (int k = 0; k < Kp; k++) {
            const float a = fabsf(r[k]);
            if (a > amax) amax = a; /* NaN never compares greater: ignored */
        }
        const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
        xs[m] = sc;
        for (int g = 0; g < G; g++) {
            int32_t sum = 0;
            for (int k = g * GROUP; k < (g + 1) * GROUP; k++) {
                float v = nearbyintf(r[k] / sc); /* default mode: ties to even */
                if (v > 127.0f) v = 127.0f;
                if (v < -127.0f) v = -127.0f;
                xq[(size_t)m * Kp + k] = (int8_t)v;
                sum += (int32_t)v;
            }
            asum[(size_t)m * G + g] = sum;
        }
    }
}

/* out[m,n,g] = sum_{k in g} (q - z) * xq  (int64, exact). zeros may be NULL (z = 8). */
void orc_group_acc(const int8_t *xq, int M, int Kp, const uint8_t *qw,
                   const uint8_t *zeros, int N, int64_t *out) {
    const int G = Kp / GROUP;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const uint8_t *row = qw + (size_t)n * (Kp / 2);
        for (int g = 0; g < G; g++) {
            const int64_t z = zeros ? zeros[(size_t)n * G + g] : 8;
            for (int m = 0; m < M; m++) {
                const int8_t *a = xq + (size_t)m * Kp;
                int64_t acc = 0;
                for (int k = g * GROUP; k < (g + 1) * GROUP; k++)
                    acc += ((int64_t)code_at(row, k, GROUP) - z) * (int64_t)a[k];
                out[((size_t)m * N + n) * G + g] = acc;
            }
        }
    }
}

/* float64 W4A16: y = sum_k x * f32((q - z) * s). absval != 0 gives |x| @ |w|^T. */
void orc_gemm_w4a16(const float *x, int M, int Kp, const uint8_t *qw,
                    const float *scales, const uint8_t *zeros, int N, double *y,
                    int absval) {
    const int G = Kp / GROUP;
#pragma omp parallel
    {
        double *w = malloc(sizeof(double) * (size_t)Kp);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            const uint8_t *row = qw + (size_t)n * (Kp / 2);
            for (int k = 0; k < Kp; k++) {
                const int g = k / GROUP;
                const float z = zeros ? (float)zeros[(size_t)n * G + g] : 8.0f;
                const float v = ((float)code_at(row, k, GROUP) - z) * scales[(size_t)n * G + g];
                w[k] = absval ? fabs((double)v) : (double)v;
            }
            for (int m = 0; m < M; m++) {
                const float *a = x + (size_t)m * Kp;
                double acc = 0.0;
                for (int k = 0; k < Kp; k++)
                    acc += (absval ? fabs((double)a[k]) : (double)a[k]) * w[k];
                y[(size_t)m * N + n] = acc;
            }
        }
        free(w);
    }
}

/* float64 MXFP4: y = sum_k x * e2m1(q) * 2^(e-127). absval as above. */
void orc_gemm_mxfp4(const float *x, int M, int Kp, const uint8_t *qw,
                    const uint8_t *e8m0, int N, double *y, int absval) {
    const int B = Kp / MXBLOCK;
#pragma omp parallel
    {
        double *w = malloc(sizeof(double) * (size_t)Kp);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            const uint8_t *row = qw + (size_t)n * (Kp / 2);
            for (int k = 0; k < Kp; k++) {
                const double v = (double)E2M1[code_at(row, k, MXBLOCK)] *
                                 (double)e8m0_f32(e8m0[(size_t)n * B + k / MXBLOCK]);
                w[k] = absval ? fabs(v) : v;
            }
            for (int m = 0; m < M; m++) {
                const float *a = x + (size_t)m * Kp;
                double acc = 0.0;
                for (int k = 0; k < Kp; k++)
                    acc += (absval ? fabs((double)a[k]) : (double)a[k]) * w[k];
                y[(size_t)m * N + n] = acc;
            }
        }
        free(w);
    }
}

/* float64 W4A8 from quantized activations: y = xs * sum_g s * acc_g.
 * bound (optional, may be NULL): xs * sum_g |s| * (sum_k q|a| + z|asum|). */
void orc_gemm_w4a8(const int8_t *xq, const float *xs, const int32_t *asum, int M,
                   int Kp, const uint8_t *qw, const float *scales,
                   const uint8_t *zeros, int N, double *y, double *bound) {
    const int G = Kp / GROUP;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const uint8_t *row = qw + (size_t)n * (Kp / 2);
        for (int m = 0; m < M; m++) {
            const int8_t *a = xq + (size_t)m * Kp;
            double tot = 0.0, mag = 0.0;
            for (int g = 0; g < G; g++) {
                const int64_t z = zeros ? zeros[(size_t)n * G + g] : 8;
                int64_t acc = 0, qa = 0;
                for (int k = g * GROUP; k < (g + 1) * GROUP; k++) {
                    const int64_t q = code_at(row, k, GROUP);
                    acc += (q - z) * (int64_t)a[k];
                    qa += q * (int64_t)(a[k] < 0 ? -a[k] : a[k]);
                }
                const double s = (double)scales[(size_t)n * G + g];
                const int64_t as = asum[(size_t)m * G + g];
                tot += s * (double)acc;
                mag += fabs(s) * ((double)qa + (double)z * (double)(as < 0 ? -as : as));
            }
            y[(size_t)m * N + n] = tot * (double)xs[m];
            if (bound) bound[(size_t)m * N + n] = mag * fabs((double)xs[m]);
        }
    }
}
