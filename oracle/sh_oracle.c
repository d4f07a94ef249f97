/* Plain-C oracle of the softhier-ops hot path -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
 *
 * A second, independent restatement of what the numpy oracle computes, used to cross-check it:
 *   - IEEE binary16 <-> binary32 conversion, round to nearest even (reference runtime/sh_rt.inc.c:31-59);
 *   - the test LCG, its fills and sample positions (runtime/sh_test.inc.c:2-39);
 *   - scalar fp32 loops for GEMM, layernorm, softmax, tanh-GELU and attention
 *     (tests/gvsoc/run.py:116-121, 152-158, 921-934).
 * Built with gcc by oracle/Makefile into oracle/liboracle.so; no GPU code, no reference sources.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- binary16 codec --------------------------------------------------------------------------------- */
float oc_h2f(uint16_t h) {
    const int sign = (h >> 15) & 1, e = (h >> 10) & 31, f = h & 1023;
    float v;
    if (e == 31) v = f ? NAN : INFINITY;
    else if (e == 0) v = ldexpf((float)f, -24);                  /* subnormal (or zero) */
    else v = ldexpf((float)(1024 + f), e - 25);                  /* (1 + f/1024) * 2^(e-15) */
    return sign ? -v : v;
}

/* Round x to binary16, nearest-even, by exact scaling: |x| = q * 2^k with an 11-bit significand q. */
uint16_t oc_f2h(float x) {
    uint16_t sign = signbit(x) ? 0x8000 : 0;
    if (isnan(x)) return sign | 0x7E00;
    float a = fabsf(x);
    if (isinf(a)) return sign | 0x7C00;
    if (a == 0.f) return sign;
    int e;
    frexpf(a, &e);                              /* a = m * 2^e, m in [0.5, 1) */
    int k = e - 11;                             /* quantum 2^k keeps 11 significant bits */
    if (k < -24) k = -24;                       /* binary16 subnormal quantum */
    double q = ldexp((double)a, -k);            /* exact in double */
    double fl = floor(q);
    double rem = q - fl;
    uint32_t n = (uint32_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (n & 1))) n++;
    /* value = n * 2^k; encode */
    if (n == 0) return sign;
    int exp = k + 10;                           /* if n in [1024, 2048): value = (n/1024) 2^(k+10) */
    if (n >= 2048) { n >>= 1; exp += 1; }       /* rounding carried into a new binade (n == 2048) */
    if (n < 1024) return sign | (uint16_t)n;    /* subnormal: k == -24 */
    if (exp > 15) return sign | 0x7C00;         /* overflow */
    return sign | (uint16_t)(((exp + 15) << 10) | (n - 1024));
}

void oc_f2h_array(const float *x, uint16_t *out, uint64_t n) { for (uint64_t i = 0; i < n; ++i) out[i] = oc_f2h(x[i]); }
void oc_h2f_array(const uint16_t *x, float *out, uint64_t n) { for (uint64_t i = 0; i < n; ++i) out[i] = oc_h2f(x[i]); }

/* ---- LCG ---------------------------------------------------------------------------------------------- */
static uint32_t lcg(uint32_t *s) { *s = *s * 1664525u + 1013904223u; return *s >> 8; }

void oc_fill_fp16(uint16_t *a, uint32_t rows, uint32_t cols, uint32_t seed, int lo, int hi, float scale) {
    uint32_t s = seed ^ 0x9E3779B9u;
    const uint32_t range = (uint32_t)(hi - lo + 1);
    for (uint64_t i = 0; i < (uint64_t)rows * cols; ++i) {
        const int v = lo + (int)(lcg(&s) % range);
        a[i] = oc_f2h((float)v * scale);
    }
}

void oc_sample_positions(uint32_t *pos, uint32_t rows, uint32_t cols, uint32_t seed, uint32_t n) {
    uint32_t s = seed ^ 0x9E3779B9u;
    for (uint32_t i = 0; i < n; ++i) { pos[2 * i] = lcg(&s) % rows; pos[2 * i + 1] = lcg(&s) % cols; }
}

/* ---- scalar references (fp32) ----------------------------------------------------------------------- */
void oc_gemm(const uint16_t *x, const uint16_t *w, float *z, uint32_t M, uint32_t N, uint32_t K) {
    for (uint32_t i = 0; i < M; ++i)
        for (uint32_t j = 0; j < N; ++j) {
            double acc = 0.0;   /* exact for short K; the tolerance absorbs fp32-vs-double differences */
            for (uint32_t k = 0; k < K; ++k) acc += (double)oc_h2f(x[(uint64_t)i * K + k]) * oc_h2f(w[(uint64_t)k * N + j]);
            z[(uint64_t)i * N + j] = (float)acc;
        }
}

void oc_layernorm(const uint16_t *x, const uint16_t *g, const uint16_t *b, float *y, uint32_t rows, uint32_t cols, float eps) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + (uint64_t)r * cols;
        double s = 0, q = 0;
        for (uint32_t c = 0; c < cols; ++c) s += oc_h2f(xr[c]);
        const double mean = s / cols;
        for (uint32_t c = 0; c < cols; ++c) { const double d = oc_h2f(xr[c]) - mean; q += d * d; }
        const double rs = 1.0 / sqrt(q / cols + eps);
        for (uint32_t c = 0; c < cols; ++c) y[(uint64_t)r * cols + c] = (float)((oc_h2f(xr[c]) - mean) * rs * oc_h2f(g[c]) + oc_h2f(b[c]));
    }
}

void oc_softmax(const uint16_t *x, float *y, uint32_t rows, uint32_t cols, float scale) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + (uint64_t)r * cols;
        double m = -INFINITY, s = 0;
        for (uint32_t c = 0; c < cols; ++c) { const double t = (double)scale * oc_h2f(xr[c]); if (t > m) m = t; }
        for (uint32_t c = 0; c < cols; ++c) s += exp((double)scale * oc_h2f(xr[c]) - m);
        for (uint32_t c = 0; c < cols; ++c) y[(uint64_t)r * cols + c] = (float)(exp((double)scale * oc_h2f(xr[c]) - m) / s);
    }
}

void oc_gelu(const uint16_t *x, float *y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        const double v = oc_h2f(x[i]);
        y[i] = (float)(0.5 * v * (1.0 + tanh(0.7978845608028654 * (v + 0.044715 * v * v * v))));
    }
}

/* One sequence: q, k, v, o are [S, D] row-major fp16; head h = columns [h dh, (h+1) dh); the fp16 roundings of
 * run.py:931-933 (scores, probabilities, output) are applied. */
void oc_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *o, uint32_t S, uint32_t D, uint32_t H, float scale) {
    const uint32_t dh = D / H;
    float *s = (float *)malloc(sizeof(float) * S);
    for (uint32_t h = 0; h < H; ++h)
        for (uint32_t i = 0; i < S; ++i) {
            float m = -INFINITY;
            for (uint32_t j = 0; j < S; ++j) {
                double acc = 0;
                for (uint32_t d = 0; d < dh; ++d) acc += (double)oc_h2f(q[(uint64_t)i * D + h * dh + d]) * oc_h2f(k[(uint64_t)j * D + h * dh + d]);
                s[j] = oc_h2f(oc_f2h((float)acc)) * scale;
                if (s[j] > m) m = s[j];
            }
            double sum = 0;
            for (uint32_t j = 0; j < S; ++j) sum += exp((double)s[j] - m);
            for (uint32_t j = 0; j < S; ++j) s[j] = oc_h2f(oc_f2h((float)(exp((double)s[j] - m) / sum)));
            for (uint32_t d = 0; d < dh; ++d) {
                double acc = 0;
                for (uint32_t j = 0; j < S; ++j) acc += (double)s[j] * oc_h2f(v[(uint64_t)j * D + h * dh + d]);
                o[(uint64_t)i * D + h * dh + d] = oc_f2h((float)acc);
            }
        }
    free(s);
}
