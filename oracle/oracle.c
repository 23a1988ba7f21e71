/* CPU oracle for the TensorPlay PrivateUse1 hot path -- TEST INFRASTRUCTURE.
 * See oracle.h for what it restates, how each function is pinned, and who
 * may call it.  Plain C99 with optional OpenMP; every value is computed in
 * double precision, rounded once to float32 (the reference's compute type)
 * and then to the storage dtype. */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- element encodings --------------------------------------------------- */

/* float -> bfloat16, round to nearest, ties to even, formulated on the value:
 * scale the significand to 7 fraction bits and round with rint() (the
 * default rounding mode is to nearest even). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    if (isnan(f)) return (uint16_t)((u >> 16) | 0x0040u);
    double a = fabs((double)f);
    if (isinf(f)) return (uint16_t)(sign | 0x7f80u);
    if (a < ldexp(1.0, -126)) { /* float subnormal: bfloat16 subnormal grid 2^-133 */
        const double q = rint(a / ldexp(1.0, -133));
        return (uint16_t)(sign | (uint16_t)q); /* q == 128 is the smallest normal */
    }
    int e;
    const double m = frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    int E = e - 1;
    double q = rint((m * 2.0 - 1.0) * 128.0);
    if (q == 128.0) {
        q = 0.0;
        E += 1;
    }
    if (E > 127) return (uint16_t)(sign | 0x7f80u);
    return (uint16_t)(sign | (uint16_t)((E + 127) << 7) | (uint16_t)q);
}

float orc_bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> IEEE binary16, round to nearest even, same formulation. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    if (isnan(f)) return (uint16_t)(sign | 0x7e00u);
    const double a = fabs((double)f);
    if (isinf(f)) return (uint16_t)(sign | 0x7c00u);
    if (a < ldexp(1.0, -14)) { /* subnormal grid 2^-24 */
        const double q = rint(a / ldexp(1.0, -24));
        return (uint16_t)(sign | (uint16_t)q); /* q == 1024 is the smallest normal */
    }
    int e;
    const double m = frexp(a, &e);
    int E = e - 1;
    double q = rint((m * 2.0 - 1.0) * 1024.0);
    if (q == 1024.0) {
        q = 0.0;
        E += 1;
    }
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((E + 15) << 10) | (uint16_t)q);
}

float orc_f16_to_f32(uint16_t h) {
    const int sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    double v;
    if (exp == 0) v = ldexp((double)man, -24);
    else if (exp == 31) v = man ? NAN : INFINITY;
    else v = ldexp(1.0 + man / 1024.0, exp - 15);
    return (float)(sign ? -v : v);
}

static double load(int dtype, const void* p, int64_t i) {
    switch (dtype) {
        case ORC_F32: return ((const float*)p)[i];
        case ORC_F16: return orc_f16_to_f32(((const uint16_t*)p)[i]);
        case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)p)[i]);
        case ORC_F64: return ((const double*)p)[i];
        case ORC_I8: return ((const int8_t*)p)[i];
        case ORC_I16: return ((const int16_t*)p)[i];
        case ORC_I32: return ((const int32_t*)p)[i];
        case ORC_I64: return (double)((const int64_t*)p)[i];
        case ORC_U8: return ((const uint8_t*)p)[i];
        case ORC_BOOL: return ((const uint8_t*)p)[i] ? 1.0 : 0.0;
    }
    return 0.0;
}

/* Round a double result to float32 (the compute type), then to ``dtype``. */
static void store_float(int dtype, void* p, int64_t i, double v) {
    const float f = (float)v;
    switch (dtype) {
        case ORC_F32: ((float*)p)[i] = f; break;
        case ORC_F16: ((uint16_t*)p)[i] = orc_f32_to_f16(f); break;
        case ORC_BF16: ((uint16_t*)p)[i] = orc_f32_to_bf16(f); break;
        case ORC_F64: ((double*)p)[i] = v; break;
    }
}

/* ---- binary arithmetic (BinaryKernels.cpp:44-87) ---------------------------- */

static double binary_value(int op, double a, double b, double alpha) {
    switch (op) {
        case 0: return a + alpha * b; /* add; sub passes -alpha (:82) */
        case 1: return a * b;
        default: return a / b;       /* CNNL_DIV_TRUE (:60-61) */
    }
}

void orc_binary(int op, int dtype, int ndim, const int64_t* sizes, const void* a,
                const int64_t* as, const void* b, const int64_t* bs, void* out,
                const int64_t* os, float alpha) {
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) n *= sizes[d];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        int64_t rem = i, oa = 0, ob = 0, oo = 0;
        for (int d = ndim - 1; d >= 0; --d) {
            const int64_t idx = rem % sizes[d];
            rem /= sizes[d];
            oa += idx * as[d];
            ob += idx * bs[d];
            oo += idx * os[d];
        }
        store_float(dtype, out, oo, binary_value(op, load(dtype, a, oa), load(dtype, b, ob), alpha));
    }
}

/* y = alpha * x + beta (cnnlTransform_v2, BinaryKernels.cpp:30-40) */
void orc_affine(int dtype, int64_t n, const void* x, float alpha, float beta, void* y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) store_float(dtype, y, i, (double)alpha * load(dtype, x, i) + beta);
}

/* ---- unary and activations (UnaryKernels.cpp:106-214) ------------------------ */

static const double kSqrt2OverPi = 0.79788456080286535587989211986876;
static const double kGeluC = 0.044715;

static double unary_value(int op, double x, double p) {
    switch (op) {
        case 0: return exp(x);
        case 1: return log(x);
        case 2: return sqrt(x);
        case 3: return 1.0 / sqrt(x);
        case 4: return -x;
        case 5: return fabs(x);
        case 6: return x * x;                               /* pow(x, 2) */
        case 7: return pow(x, p);
        case 8: return x > 0.0 ? x : 0.0;                   /* relu */
        case 9: return 1.0 / (1.0 + exp(-x));               /* sigmoid */
        case 10: return tanh(x);
        case 11: return x / (1.0 + exp(-x));                /* silu */
        case 12: return 0.5 * x * erfc(-x / sqrt(2.0));     /* gelu, erf form */
        /* gelu, tanh form: 0.5 x (1 + tanh u) = x / (1 + exp(-2u)) exactly; the
         * second form keeps full relative accuracy for large negative x */
        default: return x / (1.0 + exp(-2.0 * kSqrt2OverPi * (x + kGeluC * x * x * x)));
    }
}

void orc_unary(int op, int dtype, int64_t n, const void* x, void* y, float param) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) store_float(dtype, y, i, unary_value(op, load(dtype, x, i), param));
}

/* grad_input of the activations (UnaryKernels.cpp:222-287): threshold and
 * the input-based forms take the forward input, sigmoid and tanh the output. */
static double backward_value(int op, double g, double s, double p) {
    switch (op) {
        case 0: return s > p ? g : 0.0;
        case 1: return g * s * (1.0 - s);
        case 2: return g * (1.0 - s * s);
        case 3: {
            const double cdf = 0.5 * erfc(-s / sqrt(2.0));
            const double pdf = exp(-0.5 * s * s) / sqrt(2.0 * M_PI);
            return g * (cdf + s * pdf);
        }
        case 4: {
            /* d/dx [x sigmoid(2u)] with the same stable sigmoid */
            const double u = kSqrt2OverPi * (s + kGeluC * s * s * s);
            const double sg = 1.0 / (1.0 + exp(-2.0 * u));
            const double du = kSqrt2OverPi * (1.0 + 3.0 * kGeluC * s * s);
            return g * (sg + 2.0 * s * sg * (1.0 - sg) * du);
        }
        default: {
            const double sg = 1.0 / (1.0 + exp(-s));
            return g * sg * (1.0 + s * (1.0 - sg));
        }
    }
}

void orc_activation_backward(int op, int dtype, int64_t n, const void* grad, const void* saved,
                             void* dx, float param) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        store_float(dtype, dx, i,
                    backward_value(op, load(dtype, grad, i), load(dtype, saved, i), param));
    }
}

/* ---- reductions (ReduceKernels.cpp:21-144) ------------------------------------ */

/* max/min skipping NaN (CNNL_NOT_PROPAGATE_NAN), -0 below +0 */
static double pick(int want_max, double acc, double v, int* have) {
    if (isnan(v)) return acc;
    if (!*have) {
        *have = 1;
        return v;
    }
    if (v == acc) {
        const int v_neg = signbit(v) != 0, acc_neg = signbit(acc) != 0;
        if (want_max) return acc_neg && !v_neg ? v : acc;
        return !acc_neg && v_neg ? v : acc;
    }
    if (want_max) return v > acc ? v : acc;
    return v < acc ? v : acc;
}

void orc_reduce(int op, int dtype, int64_t outer, int64_t r, int64_t inner, const void* x,
                void* out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < outer * inner; ++t) {
        const int64_t o = t / inner, i = t % inner;
        const int64_t base = o * r * inner + i;
        double acc = 0.0;
        if (op <= 1) {
            for (int64_t j = 0; j < r; ++j) acc += load(dtype, x, base + j * inner);
            if (op == 1) acc /= (double)r;
        } else {
            int have = 0;
            acc = NAN;
            for (int64_t j = 0; j < r; ++j) acc = pick(op == 2, acc, load(dtype, x, base + j * inner), &have);
        }
        store_float(dtype, out, t, acc);
    }
}

/* ---- softmax (ReduceKernels.cpp:171-199) ---------------------------------------- */

void orc_softmax(int log_form, int dtype, int64_t outer, int64_t dim, int64_t inner,
                 const void* x, void* y) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < outer * inner; ++t) {
        const int64_t o = t / inner, i = t % inner;
        const int64_t base = o * dim * inner + i;
        double m = -INFINITY;
        for (int64_t d = 0; d < dim; ++d) {
            const double v = load(dtype, x, base + d * inner);
            if (v > m) m = v;
        }
        const double shift = isinf(m) && m < 0 ? 0.0 : m;
        double s = 0.0;
        for (int64_t d = 0; d < dim; ++d) s += exp(load(dtype, x, base + d * inner) - shift);
        const double lse = log(s);
        for (int64_t d = 0; d < dim; ++d) {
            const double v = load(dtype, x, base + d * inner) - shift;
            store_float(dtype, y, base + d * inner, log_form ? v - lse : exp(v) / s);
        }
    }
}

void orc_softmax_backward(int log_form, int dtype, int64_t outer, int64_t dim, int64_t inner,
                          const void* y, const void* dy, void* dx) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < outer * inner; ++t) {
        const int64_t o = t / inner, i = t % inner;
        const int64_t base = o * dim * inner + i;
        double s = 0.0;
        for (int64_t d = 0; d < dim; ++d) {
            const double g = load(dtype, dy, base + d * inner);
            s += log_form ? g : g * load(dtype, y, base + d * inner);
        }
        for (int64_t d = 0; d < dim; ++d) {
            const double a = load(dtype, y, base + d * inner), g = load(dtype, dy, base + d * inner);
            store_float(dtype, dx, base + d * inner, log_form ? g - exp(a) * s : a * (g - s));
        }
    }
}

/* ---- matrix products (BlasKernels.cpp:202-242) ----------------------------------- */

static double a_at(int dtype, const void* a, int64_t lda, int64_t off, int ta, int64_t i,
                   int64_t kk) {
    return load(dtype, a, off + (ta ? kk * lda + i : i * lda + kk));
}
static double b_at(int dtype, const void* b, int64_t ldb, int64_t off, int tb, int64_t kk,
                   int64_t j) {
    return load(dtype, b, off + (tb ? j * ldb + kk : kk * ldb + j));
}

static double gemm_value(int dtype, int64_t bi, int64_t i, int64_t j, int64_t k, double alpha,
                         const void* a, int64_t lda, int64_t sa, int ta, const void* b,
                         int64_t ldb, int64_t sb, int tb, double beta, const void* cin,
                         int64_t rs, int64_t cs, int64_t sbc) {
    double acc = 0.0;
    for (int64_t kk = 0; kk < k; ++kk) {
        acc += a_at(dtype, a, lda, bi * sa, ta, i, kk) * b_at(dtype, b, ldb, bi * sb, tb, kk, j);
    }
    double v = alpha * acc;
    if (beta != 0.0) v += beta * load(dtype, cin, bi * sbc + i * rs + j * cs);
    return v;
}

void orc_gemm(int dtype, int64_t batch, int64_t m, int64_t n, int64_t k, float alpha,
              const void* a, int64_t lda, int64_t sa, int ta, const void* b, int64_t ldb,
              int64_t sb, int tb, float beta, const void* cin, int64_t rs, int64_t cs,
              int64_t sbc, void* c, int64_t ldc, int64_t sc) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < batch * m; ++t) {
        const int64_t bi = t / m, i = t % m;
        for (int64_t j = 0; j < n; ++j) {
            const double v = gemm_value(dtype, bi, i, j, k, alpha, a, lda, sa, ta, b, ldb, sb,
                                        tb, beta, cin, rs, cs, sbc);
            store_float(dtype, c, bi * sc + i * ldc + j, v);
        }
    }
}

/* Exact (unrounded) values of selected entries (bij = batch, row, column
 * triples), for checking products too large to recompute whole. */
void orc_gemm_entries(int dtype, int64_t k, float alpha, const void* a, int64_t lda, int64_t sa,
                      int ta, const void* b, int64_t ldb, int64_t sb, int tb, float beta,
                      const void* cin, int64_t rs, int64_t cs, int64_t sbc, const int64_t* bij,
                      int64_t count, double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < count; ++t) {
        out[t] = gemm_value(dtype, bij[3 * t], bij[3 * t + 1], bij[3 * t + 2], k, alpha, a, lda,
                            sa, ta, b, ldb, sb, tb, beta, cin, rs, cs, sbc);
    }
}

/* ---- dtype conversion (CopyKernels.cpp:42-159) -------------------------------------- */

static int is_float_code(int d) { return d == ORC_F32 || d == ORC_F16 || d == ORC_BF16 || d == ORC_F64; }

static int64_t load_int(int dtype, const void* p, int64_t i) {
    switch (dtype) {
        case ORC_I8: return ((const int8_t*)p)[i];
        case ORC_I16: return ((const int16_t*)p)[i];
        case ORC_I32: return ((const int32_t*)p)[i];
        case ORC_I64: return ((const int64_t*)p)[i];
        case ORC_U8: return ((const uint8_t*)p)[i];
        default: return ((const uint8_t*)p)[i] ? 1 : 0;
    }
}

static void store_int(int dtype, void* p, int64_t i, int64_t v) {
    switch (dtype) {
        case ORC_I8: ((int8_t*)p)[i] = (int8_t)(uint8_t)v; break;
        case ORC_I16: ((int16_t*)p)[i] = (int16_t)(uint16_t)v; break;
        case ORC_I32: ((int32_t*)p)[i] = (int32_t)(uint32_t)v; break;
        case ORC_I64: ((int64_t*)p)[i] = v; break;
        case ORC_U8: ((uint8_t*)p)[i] = (uint8_t)v; break;
        default: ((uint8_t*)p)[i] = v != 0; break;
    }
}

/* Float to integer truncates toward zero (saturating to int64, NaN to 0) and
 * wraps to the target width; anything to bool is x != 0; integer to float
 * goes through float32 for the narrow floats.  Out-of-range conversions are
 * parity unpinned (no reference fixture fixes them). */
void orc_cast(int sd, int dd, int64_t n, const void* src, void* dst) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        if (is_float_code(sd)) {
            const double v = load(sd, src, i);
            if (is_float_code(dd)) {
                if (dd == ORC_F64) ((double*)dst)[i] = v;
                else store_float(dd, dst, i, v);
            } else if (dd == ORC_BOOL) {
                ((uint8_t*)dst)[i] = v != 0.0;
            } else {
                int64_t t;
                if (isnan(v)) t = 0;
                else if (v >= 9223372036854775807.0) t = INT64_MAX;
                else if (v <= -9223372036854775808.0) t = INT64_MIN;
                else t = (int64_t)v;
                store_int(dd, dst, i, t);
            }
        } else {
            const int64_t v = load_int(sd, src, i);
            if (dd == ORC_F64) ((double*)dst)[i] = (double)v;
            else if (is_float_code(dd)) store_float(dd, dst, i, (double)(float)v);
            else store_int(dd, dst, i, v);
        }
    }
}

/* ---- neural-network layers (NNKernels.cpp:57-395) --------------------------------- */

/* Statistics dtype of a layer norm: float32 for the 16-bit floats and
 * float32, float64 for float64 (stats_dtype, NNKernels.cpp:52-54). */
static int stats_dtype(int dtype) { return dtype == ORC_F64 ? ORC_F64 : ORC_F32; }

/* Layer norm over rows of D (NNKernels.cpp:59-100): per row the mean and the
 * biased variance, rstd = 1 / sqrt(var + eps), y = (x - mean) rstd w + b
 * (w = 1 and b = 0 when absent, :84-87).  mean and rstd are stored in the
 * statistics dtype. */
void orc_layer_norm(int dtype, int64_t rows, int64_t D, const void* x, const void* w,
                    const void* b, double eps, void* y, void* mean, void* rstd) {
    const int sd = stats_dtype(dtype);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t o = r * D;
        double s = 0.0;
        for (int64_t j = 0; j < D; ++j) s += load(dtype, x, o + j);
        const double mu = s / (double)D;
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) {
            const double d = load(dtype, x, o + j) - mu;
            ss += d * d;
        }
        const double rs = 1.0 / sqrt(ss / (double)D + eps);
        for (int64_t j = 0; j < D; ++j) {
            const double wj = w ? load(dtype, w, j) : 1.0, bj = b ? load(dtype, b, j) : 0.0;
            store_float(dtype, y, o + j, (load(dtype, x, o + j) - mu) * rs * wj + bj);
        }
        store_float(sd, mean, r, mu);
        store_float(sd, rstd, r, rs);
    }
}

/* Layer norm backward (NNKernels.cpp:104-160) from the saved statistics:
 * xhat = (x - mean) rstd, g = dy w,
 * dx = rstd (g - mean_j(g) - xhat mean_j(g xhat)),
 * dw = sum over rows of dy xhat, db = sum over rows of dy.
 * Any of dx, dw, db may be NULL (not asked for). */
void orc_layer_norm_backward(int dtype, int64_t rows, int64_t D, const void* dy, const void* x,
                             const void* mean, const void* rstd, const void* w, void* dx,
                             void* dw, void* db) {
    const int sd = stats_dtype(dtype);
    if (dx) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const int64_t o = r * D;
            const double mu = load(sd, mean, r), rs = load(sd, rstd, r);
            double sg = 0.0, sgx = 0.0;
            for (int64_t j = 0; j < D; ++j) {
                const double g = load(dtype, dy, o + j) * (w ? load(dtype, w, j) : 1.0);
                sg += g;
                sgx += g * (load(dtype, x, o + j) - mu) * rs;
            }
            const double mg = sg / (double)D, mgx = sgx / (double)D;
            for (int64_t j = 0; j < D; ++j) {
                const double g = load(dtype, dy, o + j) * (w ? load(dtype, w, j) : 1.0);
                const double xh = (load(dtype, x, o + j) - mu) * rs;
                store_float(dtype, dx, o + j, rs * (g - mg - xh * mgx));
            }
        }
    }
    if (dw || db) {
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < D; ++j) {
            double aw = 0.0, ab = 0.0;
            for (int64_t r = 0; r < rows; ++r) {
                const double g = load(dtype, dy, r * D + j);
                aw += g * (load(dtype, x, r * D + j) - load(sd, mean, r)) * load(sd, rstd, r);
                ab += g;
            }
            if (dw) store_float(dtype, dw, j, aw);
            if (db) store_float(dtype, db, j, ab);
        }
    }
}

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3", SC 2011): ten rounds; a round multiplies counter words 0
 * and 2 by the round constants into 64-bit products and recombines the
 * halves with words 1 and 3 and the key, which is bumped by the Weyl
 * constants between rounds. */
void orc_philox4x32_10(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        if (round > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* Dropout on the Philox stream (NNKernels.cpp:164-205): element e takes word
 * e % 4 of the block for counter (e / 4 as 64 bits, offset as 64 bits) under
 * key seed; its uniform (word >> 8) 2^-24 keeps it when >= p; out = x / (1 - p)
 * where kept, else 0; mask is 1 where kept. */
void orc_dropout(int dtype, int64_t n, const void* x, double p, uint64_t seed, uint64_t offset,
                 void* out, uint8_t* mask) {
    const double scale = 1.0 / (1.0 - p);
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
#pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < (n + 3) / 4; ++blk) {
        const uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)((uint64_t)blk >> 32), (uint32_t)offset,
                                 (uint32_t)(offset >> 32)};
        uint32_t word[4];
        orc_philox4x32_10(ctr, key, word);
        for (int j = 0; j < 4 && blk * 4 + j < n; ++j) {
            const int64_t e = blk * 4 + j;
            const int keep = ldexp((double)(word[j] >> 8), -24) >= p;
            mask[e] = (uint8_t)keep;
            store_float(dtype, out, e, keep ? load(dtype, x, e) * scale : 0.0);
        }
    }
}

/* out = grad * mask * scale (NNKernels.cpp:196-236). */
void orc_dropout_backward(int dtype, int64_t n, const void* grad, const uint8_t* mask,
                          double scale, void* out) {
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < n; ++e) {
        store_float(dtype, out, e, load(dtype, grad, e) * (mask[e] ? 1.0 : 0.0) * scale);
    }
}

static int64_t index_at(int index_dtype, const void* idx, int64_t i) {
    return index_dtype == ORC_I32 ? ((const int32_t*)idx)[i] : ((const int64_t*)idx)[i];
}

/* Embedding lookup (NNKernels.cpp:242-270): out[i, :] = weight[idx[i], :].
 * An index outside [0, V) gives a NaN row (the host kernel raises instead;
 * what the device returns for it is parity unpinned). */
void orc_embedding(int dtype, int64_t V, int64_t D, const void* weight, int index_dtype,
                   int64_t n, const void* idx, void* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const int64_t r = index_at(index_dtype, idx, i);
        for (int64_t j = 0; j < D; ++j) {
            store_float(dtype, out, i * D + j, r >= 0 && r < V ? load(dtype, weight, r * D + j) : NAN);
        }
    }
}

/* Dense embedding gradient (NNKernels.cpp:272-300): row r of the result is
 * the sum of dy[i, :] over the samples with idx[i] == r, each divided by the
 * number of such samples with scale_grad_by_freq; the padding row and rows
 * never indexed are zero; indices outside [0, V) add nothing. */
void orc_embedding_backward(int dtype, int64_t n, int64_t D, const void* dy, int index_dtype,
                            const void* idx, int64_t V, int64_t padding_idx,
                            int scale_grad_by_freq, void* out) {
#pragma omp parallel
    {
        double* acc = (double*)malloc((size_t)(D > 0 ? D : 1) * sizeof(double));
#pragma omp for schedule(dynamic, 16)
        for (int64_t r = 0; r < V; ++r) {
            int64_t count = 0;
            for (int64_t j = 0; j < D; ++j) acc[j] = 0.0;
            if (r != padding_idx) {
                for (int64_t i = 0; i < n; ++i) {
                    if (index_at(index_dtype, idx, i) != r) continue;
                    ++count;
                    for (int64_t j = 0; j < D; ++j) acc[j] += load(dtype, dy, i * D + j);
                }
            }
            const double scale = scale_grad_by_freq && count > 0 ? 1.0 / (double)count : 1.0;
            for (int64_t j = 0; j < D; ++j) store_float(dtype, out, r * D + j, acc[j] * scale);
        }
        free(acc);
    }
}

/* Per-sample NLL term: -w[t] x[i, t] with weight w[t]; 0 and 0 for
 * ignore_index; NaN and NaN for a target outside [0, C) (the host kernel
 * raises; parity unpinned). */
static void nll_term(int dtype, int64_t C, const void* x, int64_t i, int64_t t, const void* w,
                     int64_t ignore_index, double* loss, double* wt) {
    *loss = 0.0;
    *wt = 0.0;
    if (t == ignore_index) return;
    if (t < 0 || t >= C) {
        *loss = *wt = NAN;
        return;
    }
    *wt = w ? load(dtype, w, t) : 1.0;
    *loss = -*wt * load(dtype, x, i * C + t);
}

/* nll_loss over (N, C) with (N) targets (NNKernels.cpp:327-363): reduction 0
 * gives the per-sample terms and a zero total; 1 (mean) the sum of terms over
 * the sum of weights; 2 (sum) the sum; total is the sum of weights. */
void orc_nll_loss(int dtype, int64_t n, int64_t C, const void* x, int index_dtype,
                  const void* target, const void* w, int reduction, int64_t ignore_index,
                  void* y, void* total) {
    double sl = 0.0, sw = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        double l, wt;
        nll_term(dtype, C, x, i, index_at(index_dtype, target, i), w, ignore_index, &l, &wt);
        if (reduction == 0) store_float(dtype, y, i, l);
        sl += l;
        sw += wt;
    }
    if (reduction == 0) {
        store_float(dtype, total, 0, 0.0);
        return;
    }
    store_float(dtype, y, 0, reduction == 1 ? sl / sw : sl);
    store_float(dtype, total, 0, sw);
}

/* nll_loss backward (NNKernels.cpp:365-395): dx[i, t_i] = -w[t_i] g_i with
 * g_i = grad[i] (none), grad[0] / total (mean) or grad[0] (sum); other entries
 * 0; a NaN row for a target outside [0, C) that is not ignore_index. */
void orc_nll_loss_backward(int dtype, int64_t n, int64_t C, const void* grad, int index_dtype,
                           const void* target, const void* w, int reduction, int64_t ignore_index,
                           const void* total, void* dx) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const int64_t t = index_at(index_dtype, target, i);
        const int bad = t != ignore_index && (t < 0 || t >= C);
        double g = reduction == 0 ? load(dtype, grad, i) : load(dtype, grad, 0);
        if (reduction == 1) g /= load(dtype, total, 0);
        for (int64_t c = 0; c < C; ++c) {
            double v = 0.0;
            if (bad) v = NAN;
            else if (t != ignore_index && c == t) v = -(w ? load(dtype, w, t) : 1.0) * g;
            store_float(dtype, dx, i * C + c, v);
        }
    }
}
