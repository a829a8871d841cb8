/*
 * rmsnorm_oracle.c -- CPU restatement of cgadimpl's RMSNorm layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * The product library never links, loads or calls it, and there is no CPU
 * fallback built on it.
 *
 * What it restates (paths relative to the reference checkout):
 *   forward, rms node  cgadimpl/src/ops/normalization.cpp:23-35
 *       x2 = x*x; ms = reduce_mean(x2,{-1},keepdim); r = 1.0f/sqrt(ms+eps);
 *       xhat = x*r; tape = {r, xhat}
 *   forward, gamma     cgadimpl/src/ops/arithmetic.cpp:31-39   y = xhat*gamma
 *   backward driver    cgadimpl/src/core/autodiff.cpp:53-55,76-94
 *       root.grad = dy (assignment); reverse topological order: the Mul rule
 *       runs before the RMSNorm rule
 *   vjp_Mul            cgadimpl/src/autodiff/autodiff_vjp_ops.cpp:54-59
 *       A.grad += gy*gamma;  gamma.grad += reduce_for_broadcast(gy*xhat)
 *   reduce_for_broadcast  autodiff_vjp_ops.cpp:15-35  (sum over leading axes)
 *   vjp_RMSNorm        autodiff_vjp_ops.cpp:368-377
 *       dot = reduce_sum(gy*x,{-1},keepdim);
 *       X.grad += r*(gy - ((x*(r*r))*dot)/(float)D)
 *   accumulate_grad    cgadimpl/src/core/graph.cpp:44-47      grad += g
 *
 * Every elementwise op is evaluated in fp32, in the reference's expression
 * order, and materialised into its own buffer as the reference graph does.
 * Decisions the reference leaves open (its tensor library, OwnTensor, is not
 * in the checkout):
 *   - eps is a parameter (the reference hard-codes 1e-5f at
 *     normalization.cpp:26; the benchmark configurations use 1e-6 and 1e-5);
 *   - reductions (reduce_mean, reduce_sum) accumulate in fp64 and round the
 *     result to fp32 once; OwnTensor's accumulation order is unknowable, so
 *     parity with the GPU is to tolerance, not bitwise;
 *   - bf16 storage: inputs are widened to fp32, the fp32 path runs, outputs
 *     are rounded to bf16 round-to-nearest-even; dgamma stays fp32.
 *
 * A second, independent formulation (closed form in fp64) is provided as
 * oracle_rmsnorm_truth_f64 for the pinning checks.
 *
 * Building with -DORACLE_MUTATION=k plants deliberate mistakes (k = 1..8,
 * listed at ORACLE_MUTATION below) so the test suite can show that its
 * pinning checks catch each one.  The default build has none.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef ORACLE_MUTATION
#define ORACLE_MUTATION 0
#endif
/* Mutations (test-only builds):
 *  1  eps dropped from ms+eps
 *  2  mean divides by D-1 instead of D
 *  3  sign of the projection term in dx flipped
 *  4  dot uses the raw upstream gradient dy instead of gy = dy*gamma
 *  5  dgamma sums dy*x (r omitted)
 *  6  gamma read reversed along the hidden axis in the forward
 *  7  r*r replaced by r in dx
 *  8  dgamma omits the last row (loop bound off by one)
 */

static int g_threads = 1;

void oracle_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int oracle_get_threads(void) { return g_threads; }
int oracle_mutation(void) { return ORACLE_MUTATION; }

/* ---- bf16 storage helpers (IEEE binary32 truncated to 16 bits) ---------- */
static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN, keep sign */
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

void oracle_bf16_encode(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16_rne(in[i]);
}

void oracle_bf16_decode(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]);
}

static float* falloc(int64_t n) {
    return (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
}

/* ---- forward: rms_nodeops then mul_nodeops ------------------------------ */
/* y may alias nothing; xhat_out (nullable) receives the rms node's value.   */
int oracle_rmsnorm_fwd_f32(const float* x, const float* gamma, float* y,
                           float* inv_rms, float* xhat_out, int64_t R,
                           int64_t D, float eps) {
    if (R < 0 || D < 0) return 1;
    const int64_t N = R * D;
    if (N == 0) return 0;
    float* x2 = falloc(N);   /* x * x                      normalization.cpp:24 */
    float* ms = falloc(R);   /* reduce_mean(x2,{-1},true)  normalization.cpp:25 */
    float* t0 = falloc(R);   /* ms + eps                   normalization.cpp:26 */
    float* t1 = falloc(R);   /* sqrt(.)                                          */
    float* xhat = xhat_out ? xhat_out : falloc(N); /* x * r  normalization.cpp:27 */
    if (!x2 || !ms || !t0 || !t1 || !xhat) return 2;
    int nt = g_threads;

#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) x2[i] = x[i] * x[i];

#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) {
        double s = 0.0;
        for (int64_t j = 0; j < D; ++j) s += (double)x2[r * D + j];
#if ORACLE_MUTATION == 2
        ms[r] = (float)(s / (double)(D > 1 ? D - 1 : 1));
#else
        ms[r] = (float)(s / (double)D);
#endif
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) {
#if ORACLE_MUTATION == 1
        t0[r] = ms[r];
#else
        t0[r] = ms[r] + eps;
#endif
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) t1[r] = sqrtf(t0[r]);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) inv_rms[r] = 1.0f / t1[r];

#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) xhat[i] = x[i] * inv_rms[i / D];

    /* mul_nodeops: y = xhat * gamma (broadcast over leading axes).  Without
     * gamma the layer is ag::rms alone and y is the rms node's value.       */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        int64_t j = i % D;
#if ORACLE_MUTATION == 6
        j = D - 1 - j;
#endif
        y[i] = gamma ? xhat[i] * gamma[j] : xhat[i];
    }

    free(x2); free(ms); free(t0); free(t1);
    if (!xhat_out) free(xhat);
    return 0;
}

/* ---- backward: vjp_Mul, then vjp_RMSNorm --------------------------------- */
/* accumulate = 0: dx and dgamma start from the zero grads the Node
 * constructor allocates (graph.cpp:28-37); accumulate = 1: they hold earlier
 * gradients and receive += (graph.cpp:44-47).                              */
int oracle_rmsnorm_bwd_f32(const float* x, const float* gamma,
                           const float* inv_rms, const float* dy, float* dx,
                           float* dgamma, int64_t R, int64_t D,
                           int accumulate) {
    if (R < 0 || D < 0) return 1;
    const int64_t N = R * D;
    int nt = g_threads;
    if (N == 0) {
        if (dgamma && !accumulate)
            for (int64_t j = 0; j < D; ++j) dgamma[j] = 0.0f;
        return 0;
    }
    float* xhat = falloc(N);  /* rms node value from the tape (x*r, same op)  */
    float* gA = falloc(N);    /* rms node grad: zeros += gy*gamma              */
    float* t = falloc(N);     /* gy*xhat, input of reduce_for_broadcast        */
    float* p = falloc(N);     /* gy*x                                          */
    float* dot = falloc(R);   /* reduce_sum(p,{-1},true)                       */
    float* rr = falloc(R);    /* r*r                                           */
    float* a = falloc(N);     /* x*(r*r)                                       */
    float* b = falloc(N);     /* (.)*dot                                       */
    float* c = falloc(N);     /* (.)/D                                         */
    float* d = falloc(N);     /* gy - (.)                                      */
    float* e = falloc(N);     /* r*(.)                                         */
    if (!xhat || !gA || !t || !p || !dot || !rr || !a || !b || !c || !d || !e)
        return 2;

#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) xhat[i] = x[i] * inv_rms[i / D];

    /* vjp_Mul (autodiff_vjp_ops.cpp:54-59).  Node grads start as zeros, so
     * A.grad = 0 + gy*gamma is exactly gy*gamma.                           */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) gA[i] = gamma ? 0.0f + dy[i] * gamma[i % D] : dy[i];

    if (dgamma) {
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t i = 0; i < N; ++i) {
#if ORACLE_MUTATION == 5
            t[i] = dy[i] * x[i];
#else
            t[i] = dy[i] * xhat[i];
#endif
        }
        /* reduce_for_broadcast: sum over every leading axis (fp64 accum).   */
        int64_t rend = R;
#if ORACLE_MUTATION == 8
        rend = R - 1;
#endif
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t j = 0; j < D; ++j) {
            double s = 0.0;
            for (int64_t r = 0; r < rend; ++r) s += (double)t[r * D + j];
            float sf = (float)s;
            dgamma[j] = accumulate ? dgamma[j] + sf : 0.0f + sf;
        }
    }

    /* vjp_RMSNorm (autodiff_vjp_ops.cpp:368-377), gy = rms node grad.      */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) {
#if ORACLE_MUTATION == 4
        p[i] = dy[i] * x[i];
#else
        p[i] = gA[i] * x[i];
#endif
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) {
        double s = 0.0;
        for (int64_t j = 0; j < D; ++j) s += (double)p[r * D + j];
        dot[r] = (float)s;
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < R; ++r) {
#if ORACLE_MUTATION == 7
        rr[r] = inv_rms[r];
#else
        rr[r] = inv_rms[r] * inv_rms[r];
#endif
    }
    const float Df = (float)D;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) a[i] = x[i] * rr[i / D];
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) b[i] = a[i] * dot[i / D];
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) c[i] = b[i] / Df;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) {
#if ORACLE_MUTATION == 3
        d[i] = gA[i] + c[i];
#else
        d[i] = gA[i] - c[i];
#endif
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) e[i] = inv_rms[i / D] * d[i];
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < N; ++i) dx[i] = accumulate ? dx[i] + e[i] : 0.0f + e[i];

    free(xhat); free(gA); free(t); free(p); free(dot); free(rr);
    free(a); free(b); free(c); free(d); free(e);
    return 0;
}

/* ---- bf16 storage: widen, run the fp32 path, round outputs RNE ----------- */
int oracle_rmsnorm_fwd_bf16(const uint16_t* x, const uint16_t* gamma,
                            uint16_t* y, float* inv_rms, int64_t R, int64_t D,
                            float eps) {
    if (R < 0 || D < 0) return 1;
    const int64_t N = R * D;
    if (N == 0) return 0;
    float* xf = falloc(N);
    float* gf = gamma ? falloc(D) : NULL;
    float* yf = falloc(N);
    if (!xf || !yf || (gamma && !gf)) return 2;
    oracle_bf16_decode(x, xf, N);
    if (gamma) oracle_bf16_decode(gamma, gf, D);
    int rc = oracle_rmsnorm_fwd_f32(xf, gf, yf, inv_rms, NULL, R, D, eps);
    if (rc == 0) oracle_bf16_encode(yf, y, N);
    free(xf); free(gf); free(yf);
    return rc;
}

int oracle_rmsnorm_bwd_bf16(const uint16_t* x, const uint16_t* gamma,
                            const float* inv_rms, const uint16_t* dy,
                            uint16_t* dx, float* dgamma, int64_t R, int64_t D,
                            int accumulate) {
    if (R < 0 || D < 0) return 1;
    const int64_t N = R * D;
    if (N == 0)
        return oracle_rmsnorm_bwd_f32(NULL, NULL, NULL, NULL, NULL, dgamma, R, D,
                                      accumulate);
    float* xf = falloc(N);
    float* gf = gamma ? falloc(D) : NULL;
    float* dyf = falloc(N);
    float* dxf = falloc(N);
    if (!xf || !dyf || !dxf || (gamma && !gf)) return 2;
    oracle_bf16_decode(x, xf, N);
    if (gamma) oracle_bf16_decode(gamma, gf, D);
    oracle_bf16_decode(dy, dyf, N);
    if (accumulate) oracle_bf16_decode(dx, dxf, N);
    int rc = oracle_rmsnorm_bwd_f32(xf, gf, inv_rms, dyf, dxf, dgamma, R, D,
                                    accumulate);
    if (rc == 0) oracle_bf16_encode(dxf, dx, N);
    free(xf); free(gf); free(dyf); free(dxf);
    return rc;
}

/* ---- fp64 closed form (independent formulation) -------------------------- */
/*   ms = sum(x^2)/D, r = (ms+eps)^-1/2, y = x r gamma,
 *   g = dy gamma, dot = sum(g x), dx = r g - x r^3 dot / D,
 *   dgamma = sum_rows dy x r.                                               */
void oracle_rmsnorm_truth_f64(const double* x, const double* gamma,
                              const double* dy, double* y, double* inv_rms,
                              double* dx, double* dgamma, int64_t R, int64_t D,
                              double eps) {
    if (dgamma)
        for (int64_t j = 0; j < D; ++j) dgamma[j] = 0.0;
    for (int64_t r = 0; r < R; ++r) {
        const double* xr = x + r * D;
        double s = 0.0;
        for (int64_t j = 0; j < D; ++j) s += xr[j] * xr[j];
        double rinv = 1.0 / sqrt(s / (double)D + eps);
        if (inv_rms) inv_rms[r] = rinv;
        double dot = 0.0;
        for (int64_t j = 0; j < D; ++j) {
            double gj = gamma ? gamma[j] : 1.0;
            if (y) y[r * D + j] = xr[j] * rinv * gj;
            if (dy) dot += dy[r * D + j] * gj * xr[j];
        }
        if (!dy) continue;
        for (int64_t j = 0; j < D; ++j) {
            double gj = gamma ? gamma[j] : 1.0;
            double g = dy[r * D + j] * gj;
            if (dx) dx[r * D + j] = rinv * g - xr[j] * rinv * rinv * rinv * dot / (double)D;
            if (dgamma) dgamma[j] += dy[r * D + j] * xr[j] * rinv;
        }
    }
}
