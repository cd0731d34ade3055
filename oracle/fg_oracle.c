/*
 * fg_oracle.c -- CPU restatement of ferrograd's fused-training-path math.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); never
 * linked into the product.  Built with -ffp-contract=off so that every fp32
 * operation written here rounds exactly where it is written; fused
 * multiply-adds appear only where fmaf() is called explicitly.
 *
 * Each function cites the reference file:line whose semantics it restates;
 * paths are relative to the ferrograd repository root.
 */
#include "fg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* GELU tanh-form constants, crates/ferrograd-nn/src/op/unary.rs:493-494. */
#define GELU_C0 0.7978846f
#define GELU_C1 0.044715f

int fgo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void fgo_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------ GEMM */
/* crates/ferrograd-nn/src/op/matmul/generic.rs:98-319: C[row,col] is the
 * fmaf-accumulated sum over ascending k of A[row,k]*B[k,col] (16-wide K tiles
 * read in order, each contributing fmaf(a, b, out) for i = 0..15).  The order
 * per output element is therefore plain ascending k, which this blocked loop
 * preserves: each C element sees k-blocks in ascending order and ascending k
 * inside a block.  NT/TN index forms follow generic.rs:117-149 and :180-212. */
#define KC 256
#define NC 512
#define MB 32

void fgo_gemm(int layout, int M, int N, int K, const float *A, int lda,
              const float *B, int ldb, float *C, int ldc) {
    const float *Bp = B;
    int ldbp = ldb;
    float *packed = NULL;
    if (layout == FGO_NT) {
        /* B is stored [N][K]; pack B^T into [K][N] so the inner loop streams. */
        packed = (float *)malloc((size_t)K * (size_t)N * sizeof(float));
        if (!packed) abort();
#pragma omp parallel for schedule(static)
        for (int k = 0; k < K; ++k)
            for (int j = 0; j < N; ++j) packed[(size_t)k * N + j] = B[(size_t)j * ldb + k];
        Bp = packed;
        ldbp = N;
    }
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i)
        memset(C + (size_t)i * ldc, 0, (size_t)N * sizeof(float));

    const int nmb = (M + MB - 1) / MB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int ib = 0; ib < nmb; ++ib) {
        const int i0 = ib * MB, i1 = (i0 + MB < M) ? i0 + MB : M;
        for (int j0 = 0; j0 < N; j0 += NC) {
            const int j1 = (j0 + NC < N) ? j0 + NC : N;
            for (int k0 = 0; k0 < K; k0 += KC) {
                const int k1 = (k0 + KC < K) ? k0 + KC : K;
                for (int i = i0; i < i1; ++i) {
                    float *c = C + (size_t)i * ldc;
                    for (int k = k0; k < k1; ++k) {
                        const float a = (layout == FGO_TN) ? A[(size_t)k * lda + i]
                                                           : A[(size_t)i * lda + k];
                        const float *b = Bp + (size_t)k * ldbp;
                        for (int j = j0; j < j1; ++j) c[j] = fmaf(a, b[j], c[j]);
                    }
                }
            }
        }
    }
    free(packed);
}

/* ----------------------------------------------------------- activations */
/* ReLU forward max(x, 0): unary.rs:449.  Backward mask [z > 0]: the
 * reference's mask (unary.rs:460-469) reads the node's own output and tests
 * >= 0, which never blocks; the derivative used here is the correct one,
 * with 0 at z == 0 (PyTorch convention). */
static inline double act_d(int act, double z) {
    if (act == FGO_ACT_RELU) return z > 0.0 ? z : 0.0;
    if (act == FGO_ACT_GELU) {
        /* unary.rs:501-587: 0.5*x*(1 + tanh(0.7978846*(x + 0.044715*x^3))) */
        const double u = (double)GELU_C0 * (z + (double)GELU_C1 * z * z * z);
        return 0.5 * z * (1.0 + tanh(u));
    }
    return z;
}

static inline double act_grad_d(int act, double z) {
    if (act == FGO_ACT_RELU) return z > 0.0 ? 1.0 : 0.0;
    if (act == FGO_ACT_GELU) {
        /* d/dz of the tanh form (the reference's unary.rs:588-714 evaluates
         * this with tanh(u) in place of z -- corrected). */
        const double c0 = (double)GELU_C0, c1 = (double)GELU_C1;
        const double u = c0 * (z + c1 * z * z * z);
        const double t = tanh(u);
        return 0.5 * (1.0 + t) + 0.5 * z * (1.0 - t * t) * c0 * (1.0 + 3.0 * c1 * z * z);
    }
    return 1.0;
}

float fgo_act(int act, float z) { return (float)act_d(act, (double)z); }
float fgo_act_grad(int act, float z) { return (float)act_grad_d(act, (double)z); }

void fgo_bias_act(int M, int N, const float *C, int ldc, const float *bias,
                  int act, float *Z, float *H) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            const float z = C[(size_t)i * ldc + j] + (bias ? bias[j] : 0.0f);
            if (Z) Z[(size_t)i * N + j] = z;
            if (H) H[(size_t)i * N + j] = (float)act_d(act, (double)z);
        }
    }
}

void fgo_act_bwd(int act, int64_t n, const float *dH, const float *Z, float *dZ) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        dZ[i] = (float)((double)dH[i] * act_grad_d(act, (double)Z[i]));
}

void fgo_bias_grad(int M, int N, const float *dZ, int ld, float *dbias) {
#pragma omp parallel for schedule(static)
    for (int j = 0; j < N; ++j) {
        double s = 0.0;
        for (int i = 0; i < M; ++i) s += (double)dZ[(size_t)i * ld + j];
        dbias[j] = (float)s;
    }
}

/* --------------------------------------------------------- softmax + CE */
/* softmax.rs:112-446: per row, max over columns, e = exp(x - max), sum,
 * scale by 1/sum.  basic_loss.rs:91-133: label = labels[row] (u32);
 * loss = -log(p[label]); grad = p - [col == label].  Here the loss is taken
 * as lse - x[label] (identical in exact arithmetic, finite when p underflows)
 * and the gradient is written for the logits directly. */
double fgo_softmax_ce(int R, int C, const float *x, int ldx, const uint32_t *labels,
                      float grad_scale, float *row_loss, float *dlogits,
                      int ldd, uint32_t *argmax) {
    double total = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : total)
    for (int r = 0; r < R; ++r) {
        const float *xr = x + (size_t)r * ldx;
        float m = xr[0];
        uint32_t am = 0;
        for (int c = 1; c < C; ++c)
            if (xr[c] > m) { m = xr[c]; am = (uint32_t)c; }
        double s = 0.0;
        for (int c = 0; c < C; ++c) s += (double)expf(xr[c] - m);
        const double lse = (double)m + log(s);
        const uint32_t t = labels ? labels[r] : 0u;
        const double loss = lse - (double)xr[t];
        if (row_loss) row_loss[r] = (float)loss;
        if (argmax) argmax[r] = am;
        total += loss;
        if (dlogits) {
            float *dr = dlogits + (size_t)r * ldd;
            for (int c = 0; c < C; ++c) {
                const double p = (double)expf(xr[c] - m) / s;
                dr[c] = (float)((double)grad_scale * (p - ((uint32_t)c == t ? 1.0 : 0.0)));
            }
        }
    }
    return R > 0 ? total / (double)R : 0.0;
}

void fgo_softmax(int R, int C, const float *x, float *y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < R; ++r) {
        const float *xr = x + (size_t)r * C;
        float m = xr[0];
        for (int c = 1; c < C; ++c) m = xr[c] > m ? xr[c] : m;
        double s = 0.0;
        for (int c = 0; c < C; ++c) s += (double)expf(xr[c] - m);
        for (int c = 0; c < C; ++c) y[(size_t)r * C + c] = (float)((double)expf(xr[c] - m) / s);
    }
}

/* softmax.rs:448-688: dot = sum dy*y; dx = y*(dy - dot), over all columns. */
void fgo_softmax_bwd(int R, int C, const float *y, const float *dy, float *dx) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < R; ++r) {
        const float *yr = y + (size_t)r * C, *dyr = dy + (size_t)r * C;
        double dot = 0.0;
        for (int c = 0; c < C; ++c) dot += (double)dyr[c] * (double)yr[c];
        for (int c = 0; c < C; ++c)
            dx[(size_t)r * C + c] = (float)((double)yr[c] * ((double)dyr[c] - dot));
    }
}

/* ------------------------------------------------------------ optimisers */
/* crates/ferrograd-nn/src/optim/basic_optim.rs:3-31: scaled = g * lr
 * (Op::Mul), weight -= scaled (param_sub), grad = 0 (param_store). */
void fgo_sgd(int64_t n, float *w, float *g, float lr, int zero_grad) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float scaled = g[i] * lr;
        w[i] = w[i] - scaled;
        if (zero_grad) g[i] = 0.0f;
    }
}

void fgo_adam_scalars(double lr, double b1, double b2, int step,
                      float *step_size, float *inv_sqrt_bc2) {
    const double bc1 = 1.0 - pow(b1, (double)step);
    const double bc2 = 1.0 - pow(b2, (double)step);
    *step_size = (float)(lr / bc1);
    *inv_sqrt_bc2 = (float)(1.0 / sqrt(bc2));
}

void fgo_adam(int64_t n, float *p, const float *g, float *m, float *v,
              float b1, float b2, float eps, float step_size,
              float inv_sqrt_bc2) {
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float gi = g[i];
        const float mi = b1 * m[i] + omb1 * gi;
        const float vi = b2 * v[i] + omb2 * (gi * gi);
        const float denom = sqrtf(vi) * inv_sqrt_bc2 + eps;
        p[i] = p[i] - (step_size * mi) / denom;
        m[i] = mi;
        v[i] = vi;
    }
}

/* ------------------------------------------------ 16-bit storage types */
uint16_t fgo_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) /* infinity, or NaN (quieted, top payload bits kept) */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u | ((a >> 13) & 0x3ffu) : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                                   /* below 2^-14: subnormal or zero */
        if (a < 0x33000000u) return sign;                    /* <= 2^-25 rounds to zero */
        const uint32_t e = a >> 23;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e; /* value = m * 2^(e-150) = (m >> shift) units of 2^-24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    const uint32_t e = (a >> 23) - 127u + 15u;
    const uint32_t m = a & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* carry may reach infinity */
    return (uint16_t)(sign | q);
}

float fgo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        float f = ldexpf((float)m, -24); /* exact: m < 2^10 */
        memcpy(&u, &f, 4);
        u |= sign;
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t fgo_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float fgo_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float to_f(int dt, uint16_t h) {
    return dt == FGO_BF16 ? fgo_bf16_to_f32(h) : fgo_f16_to_f32(h);
}
static inline uint16_t from_f(int dt, float f) {
    return dt == FGO_BF16 ? fgo_f32_to_bf16(f) : fgo_f32_to_f16(f);
}
static inline float rnd(int dt, float f) { return to_f(dt, from_f(dt, f)); }

void fgo_to_f32(int dtype, int64_t n, const uint16_t *src, float *dst) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) dst[i] = to_f(dtype, src[i]);
}

void fgo_from_f32(int dtype, int64_t n, const float *src, uint16_t *dst) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) dst[i] = from_f(dtype, src[i]);
}

/* Widen a rows x cols operand with leading dimension ld into a dense array. */
static float *widen(int dt, int rows, int cols, const uint16_t *src, int ld) {
    float *d = (float *)malloc((size_t)(rows > 0 ? rows : 1) * (size_t)(cols > 0 ? cols : 1) * 4);
    if (!d) abort();
#pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; ++i)
        for (int j = 0; j < cols; ++j) d[(size_t)i * cols + j] = to_f(dt, src[(size_t)i * ld + j]);
    return d;
}

static float *gemm_x16_sum(int dt, int layout, int M, int N, int K, const uint16_t *A, int lda,
                           const uint16_t *B, int ldb) {
    const int ar = layout == FGO_TN ? K : M, ac = layout == FGO_TN ? M : K;
    const int br = layout == FGO_NT ? N : K, bc = layout == FGO_NT ? K : N;
    float *a = widen(dt, ar, ac, A, lda);
    float *b = widen(dt, br, bc, B, ldb);
    float *s = (float *)malloc((size_t)(M > 0 ? M : 1) * (size_t)(N > 0 ? N : 1) * 4);
    if (!s) abort();
    fgo_gemm(layout, M, N, K, a, ac, b, bc, s, N);
    free(a);
    free(b);
    return s;
}

void fgo_gemm_x16(int dtype, int layout, int M, int N, int K,
                  const uint16_t *A, int lda, const uint16_t *B, int ldb,
                  const uint16_t *bias, int act, uint16_t *C, int ldc,
                  uint16_t *Z, int ldz, int accumulate) {
    float *s = gemm_x16_sum(dtype, layout, M, N, K, A, lda, B, ldb);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            float v = rnd(dtype, s[(size_t)i * N + j]);
            if (bias) v = rnd(dtype, v + to_f(dtype, bias[j]));
            if (Z) Z[(size_t)i * ldz + j] = from_f(dtype, v);
            float o = act == FGO_ACT_NONE ? v : rnd(dtype, (float)act_d(act, (double)v));
            if (accumulate) o = o + to_f(dtype, C[(size_t)i * ldc + j]);
            C[(size_t)i * ldc + j] = from_f(dtype, o);
        }
    }
    free(s);
}

void fgo_gemm_bwd_x16(int dtype, int layout, int M, int N, int K,
                      const uint16_t *A, int lda, const uint16_t *B, int ldb,
                      int act, const uint16_t *Zs, int ldzs, uint16_t *C,
                      int ldc, int accumulate) {
    float *s = gemm_x16_sum(dtype, layout, M, N, K, A, lda, B, ldb);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            float v = rnd(dtype, s[(size_t)i * N + j]);
            if (act != FGO_ACT_NONE) {
                const float z = to_f(dtype, Zs[(size_t)i * ldzs + j]);
                /* ReLU' masks the gradient (0 where z <= 0, as the reference's
                 * conditional add leaves it); GELU' scales it. */
                v = act == FGO_ACT_RELU ? (z > 0.0f ? v : 0.0f)
                                        : rnd(dtype, v * (float)act_grad_d(act, (double)z));
            }
            if (accumulate) v = v + to_f(dtype, C[(size_t)i * ldc + j]);
            C[(size_t)i * ldc + j] = from_f(dtype, v);
        }
    }
    free(s);
}
