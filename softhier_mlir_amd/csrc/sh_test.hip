// Test helpers of the reference library (runtime/sh_test.inc.c:2-115): LCG fills, sampled dumps in the
// "<tag> r c hex" text protocol, the sampled GEMM self-check and constant fills/checks.
//
// The LCG is s <- s * 1664525 + 1013904223 (mod 2^32), s0 = seed ^ 0x9E3779B9, output s >> 8 (the
// reference's sh_lcg, sh_test.inc.c:2). Element n of a fill (row-major over rows x cols) takes output
// n + 1; on the GPU each thread jumps straight to its first element by composing the affine step map
// (x -> a x + c) with itself in O(log n) and then steps sequentially, so the values equal the sequential loop.
#include "sh_common.h"
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kLcgA = 1664525u, kLcgC = 1013904223u, kSeedMix = 0x9E3779B9u;
constexpr uint32_t kFillRun = 16;     // consecutive elements per thread

__host__ __device__ inline uint32_t lcg_next(uint32_t &s) { s = s * kLcgA + kLcgC; return s >> 8; }

// state after k steps from s0
__device__ inline uint32_t lcg_jump(uint32_t s0, uint64_t k) {
    uint32_t ra = 1u, rc = 0u, ba = kLcgA, bc = kLcgC;
    while (k) {
        if (k & 1) { rc = ba * rc + bc; ra = ba * ra; }
        bc = ba * bc + bc; ba = ba * ba;
        k >>= 1;
    }
    return ra * s0 + rc;
}

__global__ void k_fill_lcg(uint16_t *a, uint32_t rows, uint32_t cols, uint64_t ld, uint32_t s0, int lo, uint32_t range, float scale) {
    const uint64_t total = (uint64_t)rows * cols;
    const uint64_t n0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * kFillRun;
    if (n0 >= total) return;
    uint32_t s = lcg_jump(s0, n0);                 // state before element n0
    uint32_t r = (uint32_t)(n0 / cols), c = (uint32_t)(n0 % cols);
    for (uint32_t i = 0; i < kFillRun && n0 + i < total; ++i) {
        const int v = lo + (int)(lcg_next(s) % range);
        a[(uint64_t)r * ld + c] = sh_dev_f2h((float)v * scale);
        if (++c == cols) { c = 0; ++r; }
    }
}

__global__ void k_fill_bits(uint16_t *a, uint32_t rows, uint32_t cols, uint64_t ld, uint16_t even, uint16_t odd) {
    const uint64_t n = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= (uint64_t)rows * cols) return;
    const uint32_t r = (uint32_t)(n / cols), c = (uint32_t)(n % cols);
    a[(uint64_t)r * ld + c] = (c & 1) ? odd : even;
}

__global__ void k_count_near(const uint16_t *a, uint32_t rows, uint32_t cols, uint64_t ld, int bits, int tol, uint32_t *ok) {
    const uint64_t n = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool hit = false;
    if (n < (uint64_t)rows * cols) {
        const uint32_t r = (uint32_t)(n / cols), c = (uint32_t)(n % cols);
        int d = (int)a[(uint64_t)r * ld + c] - bits;
        if (d < 0) d = -d;
        hit = d <= tol;
    }
    const unsigned long long m = __ballot(hit);
    if ((threadIdx.x & 63) == 0 && m) atomicAdd(ok, (uint32_t)__popcll(m));
}

__global__ void k_gather(uint16_t *out, const uint16_t *a, const uint32_t *pos, uint32_t n, uint64_t ld) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[(uint64_t)pos[2 * i] * ld + pos[2 * i + 1]];
}

// One thread per sample: acc = z0 + sum_k x[i,k] w[k,j] in fp32, k ascending (sh_test.inc.c:41-43).
__global__ void k_check_dots(float *want, uint16_t *got, const uint16_t *x, const uint16_t *w, const uint16_t *z,
                             const uint32_t *pos, uint32_t n, uint32_t K, uint64_t ldx, uint64_t ldw, uint64_t ldz, float z0) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const uint32_t i = pos[2 * t], j = pos[2 * t + 1];
    float acc = z0;
    for (uint32_t k = 0; k < K; ++k) acc += sh_dev_h2f(x[(uint64_t)i * ldx + k]) * sh_dev_h2f(w[(uint64_t)k * ldw + j]);
    want[t] = acc;
    got[t] = z[(uint64_t)i * ldz + j];
}

// Device staging for the helpers (separate from the GEMM workspace so neither resizes the other).
void *small_buf(size_t bytes) {
    static void *p = nullptr;
    static size_t have = 0;
    if (bytes <= have) return p;
    if (p) { sh_barrier_global(); (void)hipFree(p); p = nullptr; have = 0; }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (!sh_hip_ok(hipMalloc(&p, want), "test helper hipMalloc")) { p = nullptr; return nullptr; }
    have = want;
    return p;
}

bool addr_ok(const char *op, uint64_t a) {
    if (!a) { sh_set_error(-1, "[%s] NULL tensor address", op); return false; }
    sh_ensure_init();
    return true;
}

// Gather `pos` ((i, j) pairs) of a [*, ld] fp16 matrix to the host.
bool gather(const char *op, uint64_t a, uint64_t ld, const std::vector<uint32_t> &pos, std::vector<uint16_t> &out) {
    const uint32_t n = (uint32_t)(pos.size() / 2);
    out.assign(n, 0);
    if (!n) return true;
    char *buf = (char *)small_buf((size_t)n * 8 + (size_t)n * 2 + 256);
    if (!buf) return false;
    uint32_t *dpos = (uint32_t *)buf;
    uint16_t *dout = (uint16_t *)(buf + (size_t)n * 8);
    hipStream_t st = sh_stream();
    if (!sh_hip_ok(hipMemcpyAsync(dpos, pos.data(), (size_t)n * 8, hipMemcpyHostToDevice, st), op)) return false;
    hipLaunchKernelGGL(k_gather, dim3(sh_cdiv(n, 256)), dim3(256), 0, st, dout, (const uint16_t *)a, dpos, n, ld);
    if (!sh_launch_ok(op)) return false;
    if (!sh_hip_ok(hipMemcpyAsync(out.data(), dout, (size_t)n * 2, hipMemcpyDeviceToHost, st), op)) return false;
    return sh_hip_ok(hipStreamSynchronize(st), op);
}

void fill_lcg(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, int lo, int hi, float scale) {
    if (!addr_ok("sh_test_fill_fp16", a) || !rows || !cols) return;
    const uint64_t total = (uint64_t)rows * cols;
    const uint64_t threads = (total + kFillRun - 1) / kFillRun;
    hipLaunchKernelGGL(k_fill_lcg, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, sh_stream(), (uint16_t *)a, rows, cols,
                       (uint64_t)ld, seed ^ kSeedMix, lo, (uint32_t)(hi - lo + 1), scale);
    sh_launch_ok("sh_test_fill_fp16");
}

void fill_bits(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t even, uint32_t odd) {
    if (!addr_ok("sh_test_fill_const_fp16", a) || !rows || !cols) return;
    const uint64_t total = (uint64_t)rows * cols;
    hipLaunchKernelGGL(k_fill_bits, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, sh_stream(), (uint16_t *)a, rows, cols,
                       (uint64_t)ld, (uint16_t)even, (uint16_t)odd);
    sh_launch_ok("sh_test_fill_const_fp16");
}

}  // namespace

extern "C" {

void sh_test_fill_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, int lo, int hi, float scale) {
    fill_lcg(a, rows, cols, ld, seed, lo, hi, scale);
}
void sh_test_fill_int_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, int lo, int hi) {
    fill_lcg(a, rows, cols, ld, seed, lo, hi, 1.0f);
}

void sh_test_dump_samples(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, uint32_t nsamples, const char *tag) {
    if (!addr_ok("sh_test_dump_samples", a) || !rows || !cols) return;
    uint32_t s = seed ^ kSeedMix;
    std::vector<uint32_t> pos(2 * (size_t)nsamples);
    for (uint32_t n = 0; n < nsamples; ++n) {
        pos[2 * n] = lcg_next(s) % rows;
        pos[2 * n + 1] = lcg_next(s) % cols;
    }
    std::vector<uint16_t> v;
    if (!gather("sh_test_dump_samples", a, ld, pos, v)) return;
    std::string out;
    char line[256];
    for (uint32_t n = 0; n < nsamples; ++n) {
        snprintf(line, sizeof line, "%s %u %u %04x\n", tag ? tag : "", pos[2 * n], pos[2 * n + 1], (uint32_t)v[n]);
        out += line;
    }
    sh_printf("%s", out.c_str());
}

void sh_test_dump_samples_idx(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t seed, uint32_t nsamples, const char *tag, uint32_t idx) {
    char t[64];
    snprintf(t, sizeof t, "%s%u", tag ? tag : "", idx);
    sh_test_dump_samples(a, rows, cols, ld, seed, nsamples, t);
}

void sh_test_dump_all(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, const char *tag) {
    if (!addr_ok("sh_test_dump_all", a) || !rows || !cols) return;
    std::vector<uint16_t> h((size_t)rows * cols);
    sh_barrier_global();
    if (!sh_hip_ok(hipMemcpy2D(h.data(), (size_t)cols * 2, (const void *)a, (size_t)ld * 2, (size_t)cols * 2, rows, hipMemcpyDeviceToHost),
                   "sh_test_dump_all")) return;
    std::string out;
    char line[256];
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < cols; ++c) {
            snprintf(line, sizeof line, "%s %u %u %04x\n", tag ? tag : "", r, c, (uint32_t)h[(size_t)r * cols + c]);
            out += line;
        }
    sh_printf("%s", out.c_str());
}

void sh_test_dump_all_idx(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, const char *tag, uint32_t idx) {
    char t[64];
    snprintf(t, sizeof t, "%s%u", tag ? tag : "", idx);
    sh_test_dump_all(a, rows, cols, ld, t);
}

uint32_t sh_test_check_gemm(uint64_t x, uint64_t w, uint64_t z, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t ldx, uint32_t ldw, uint32_t ldz, uint32_t nsamples, float tol, float z0, const char *tag) {
    if (!addr_ok("sh_test_check_gemm", x) || !addr_ok("sh_test_check_gemm", w) || !addr_ok("sh_test_check_gemm", z)) return nsamples;
    if (!M || !N || !nsamples) return 0;
    uint32_t s = 0xC0FFEEu;
    std::vector<uint32_t> pos(2 * (size_t)nsamples);
    for (uint32_t n = 0; n < nsamples; ++n) {      // sh_test.inc.c:38-39: strided grid plus LCG jitter
        const uint32_t j1 = lcg_next(s);
        pos[2 * n] = (n * 7919u + j1) % M;
        const uint32_t j2 = lcg_next(s);
        pos[2 * n + 1] = (n * 104729u + j2) % N;
    }
    char *buf = (char *)small_buf((size_t)nsamples * 14 + 256);
    if (!buf) return nsamples;
    uint32_t *dpos = (uint32_t *)buf;
    float *dwant = (float *)(buf + (size_t)nsamples * 8);
    uint16_t *dgot = (uint16_t *)(buf + (size_t)nsamples * 12);
    hipStream_t st = sh_stream();
    std::vector<float> want(nsamples);
    std::vector<uint16_t> got(nsamples);
    if (!sh_hip_ok(hipMemcpyAsync(dpos, pos.data(), (size_t)nsamples * 8, hipMemcpyHostToDevice, st), "sh_test_check_gemm")) return nsamples;
    hipLaunchKernelGGL(k_check_dots, dim3(sh_cdiv(nsamples, 64)), dim3(64), 0, st, dwant, dgot, (const uint16_t *)x, (const uint16_t *)w,
                       (const uint16_t *)z, dpos, nsamples, K, (uint64_t)ldx, (uint64_t)ldw, (uint64_t)ldz, z0);
    if (!sh_launch_ok("sh_test_check_gemm")) return nsamples;
    sh_hip_ok(hipMemcpyAsync(want.data(), dwant, (size_t)nsamples * 4, hipMemcpyDeviceToHost, st), "sh_test_check_gemm");
    sh_hip_ok(hipMemcpyAsync(got.data(), dgot, (size_t)nsamples * 2, hipMemcpyDeviceToHost, st), "sh_test_check_gemm");
    if (!sh_hip_ok(hipStreamSynchronize(st), "sh_test_check_gemm")) return nsamples;
    uint32_t bad = 0;
    float maxdiff = 0.f;
    for (uint32_t n = 0; n < nsamples; ++n) {
        const float g = sh_fp16_to_f32(got[n]);
        float d = g - want[n];
        if (d < 0) d = -d;
        if (d > maxdiff) maxdiff = d;
        if (d > tol) {
            if (bad < 4) sh_printf("  mismatch z[%u,%u] got %f want %f\n", pos[2 * n], pos[2 * n + 1], g, want[n]);
            ++bad;
        }
    }
    sh_printf("%s samples=%u bad=%u maxdiff=%f %s\n", tag ? tag : "", nsamples, bad, maxdiff, bad ? "FAIL" : "PASS");
    return bad;
}

void sh_test_fill_const_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t bits) {
    fill_bits(a, rows, cols, ld, bits, bits);
}

void sh_test_fill_colparity_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t even, uint32_t odd) {
    fill_bits(a, rows, cols, ld, even, odd == 0xFFFFFFFFu ? even : odd);
}

uint32_t sh_test_check_const_fp16(uint64_t a, uint32_t rows, uint32_t cols, uint32_t ld, uint32_t bits, uint32_t tol, const char *tag) {
    if (!addr_ok("sh_test_check_const_fp16", a)) return 0;
    uint32_t ok = 0;
    const uint64_t total = (uint64_t)rows * cols;
    if (total) {
        uint32_t *cnt = (uint32_t *)small_buf(256);
        if (!cnt) return 0;
        hipStream_t st = sh_stream();
        hipLaunchKernelGGL(k_fill_bits, dim3(1), dim3(64), 0, st, (uint16_t *)cnt, 1u, 2u, (uint64_t)2, (uint16_t)0, (uint16_t)0);
        hipLaunchKernelGGL(k_count_near, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, st, (const uint16_t *)a, rows, cols,
                           (uint64_t)ld, (int)(bits & 0xFFFFu), (int)tol, cnt);
        if (!sh_launch_ok("sh_test_check_const_fp16")) return 0;
        sh_hip_ok(hipMemcpyAsync(&ok, cnt, 4, hipMemcpyDeviceToHost, st), "sh_test_check_const_fp16");
        sh_hip_ok(hipStreamSynchronize(st), "sh_test_check_const_fp16");
    }
    sh_printf("%s_CHECK ok=%u/%u %s_%s\n", tag ? tag : "", ok, rows * cols, tag ? tag : "", ok == rows * cols ? "PASS" : "FAIL");
    return ok;
}

}  // extern "C"
